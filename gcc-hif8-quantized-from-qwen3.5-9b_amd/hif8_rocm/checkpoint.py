"""Reading an exported HiFloat8 static checkpoint (W8A8HIF8_STATIC + KV8).

Format (docs/checkpoint-format.md:5-57; written by exporter.py:700-762):

* safetensors shards (``model.safetensors`` or an index
  ``model.safetensors.index.json``) holding, per quantised Linear component
  ``<name>``: ``<name>.weight`` U8 ``[N, K]``, ``<name>.weight_scale`` F32
  ``[N, 1]`` and ``<name>.input_scale`` F32 ``[1]``; other tensors in their
  float dtype;
* ``quant_model_description.json``: tensor name -> ``W8A8HIF8_STATIC`` (Linear
  weights), ``W8A8HIF8_SOFT`` (the token embedding: rows + scales, no
  activation quantisation) or ``FLOAT``;
* ``hif8_metadata.json``: ``format``, and for static checkpoints
  ``kv_cache = {"mode": "static_per_layer_per_head", "layers": {"<i>":
  {"key_scales": [...], "value_scales": [...]}}}``.

Fused runtime Linears (``qkv_proj`` = q+k+v, ``gate_up_proj`` = gate+up,
``in_proj_qkvz`` = qkv+z) are built by concatenating their components' rows;
the components share one activation scale (the exporter writes one
normalised input scale per fused group), which is checked.
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Sequence

import torch

from . import scheme

QUANT_DESCRIPTION_FILENAME = "quant_model_description.json"
METADATA_FILENAME = "hif8_metadata.json"
STATIC_QUANT_TYPE = scheme.STATIC_QUANT_TYPE
SOFT_QUANT_TYPE = scheme.SOFT_QUANT_TYPE
FLOAT_TYPE = "FLOAT"
KV_MODE = "static_per_layer_per_head"


def load_static_kv_scales(checkpoint: str | Path) -> dict[int, tuple[tuple[float, ...], tuple[float, ...]]] | None:
    """Per-layer, per-head static K/V scales of a checkpoint (kv_runtime.py:205-264).

    A checkpoint without metadata, or a dynamic one without ``kv_cache``,
    gives None.  A static checkpoint is fail-closed: missing or malformed
    scales raise ValueError rather than falling back to runtime scales.
    """
    directory = Path(checkpoint)
    path = directory / METADATA_FILENAME
    if not path.is_file():
        return None
    metadata = json.loads(path.read_text(encoding="utf-8"))
    if not isinstance(metadata, dict):
        raise ValueError(f"invalid HIF8 metadata object: {path}")
    kv_cache = metadata.get("kv_cache")
    if kv_cache is None:
        if metadata.get("format") == STATIC_QUANT_TYPE:
            raise ValueError(f"static HIF8 checkpoint is missing kv_cache metadata: {path}")
        return None
    if not isinstance(kv_cache, dict) or kv_cache.get("mode") != KV_MODE:
        raise ValueError(f"unsupported HIF8 kv_cache metadata in {path}")
    layers = kv_cache.get("layers")
    if not isinstance(layers, dict) or not layers:
        raise ValueError(f"HIF8 kv_cache.layers is empty in {path}")
    out: dict[int, tuple[tuple[float, ...], tuple[float, ...]]] = {}
    for raw, entry in layers.items():
        try:
            index = int(raw)
        except (TypeError, ValueError) as error:
            raise ValueError(f"invalid static KV layer index {raw!r}") from error
        if str(index) != str(raw) or index < 0:
            raise ValueError(f"invalid static KV layer index {raw!r}")
        if not isinstance(entry, dict):
            raise ValueError(f"static KV layer {index} is not an object")
        pair = []
        for kind in ("key_scales", "value_scales"):
            values = entry.get(kind)
            if not isinstance(values, list) or not values:
                raise ValueError(f"static KV layer {index} has no {kind}")
            scales = tuple(float(v) for v in values)
            if any(not math.isfinite(v) or v <= 0.0 for v in scales):
                raise ValueError(f"static KV layer {index} has invalid {kind}")
            pair.append(scales)
        if len(pair[0]) != len(pair[1]):
            raise ValueError(f"static KV layer {index} has different K/V head counts")
        out[index] = (pair[0], pair[1])
    return out


@dataclass
class Hif8Checkpoint:
    """An opened checkpoint directory: tensor index, quant description, metadata."""

    path: Path
    weight_map: dict[str, str]
    description: dict[str, str]
    metadata: dict[str, Any]
    _handles: dict[str, Any] = field(default_factory=dict, repr=False)

    @classmethod
    def open(cls, path: str | Path) -> "Hif8Checkpoint":
        directory = Path(path)
        weight_map = _weight_map(directory)
        desc_path = directory / QUANT_DESCRIPTION_FILENAME
        if not desc_path.is_file():
            raise FileNotFoundError(f"missing {QUANT_DESCRIPTION_FILENAME} in {directory}")
        description = json.loads(desc_path.read_text(encoding="utf-8"))
        if not isinstance(description, dict):
            raise ValueError(f"invalid quant description: {desc_path}")
        allowed = {STATIC_QUANT_TYPE, SOFT_QUANT_TYPE, FLOAT_TYPE}
        bad = sorted({str(v) for v in description.values()} - allowed)
        if bad:
            raise ValueError(f"unsupported quant types in {desc_path}: {bad}")
        meta_path = directory / METADATA_FILENAME
        metadata = json.loads(meta_path.read_text(encoding="utf-8")) if meta_path.is_file() else {}
        if not isinstance(metadata, dict):
            raise ValueError(f"invalid HIF8 metadata object: {meta_path}")
        if metadata and metadata.get("format") not in (STATIC_QUANT_TYPE, SOFT_QUANT_TYPE):
            raise ValueError(f"{meta_path} declares unsupported format {metadata.get('format')!r}")
        return cls(directory, weight_map, {str(k): str(v) for k, v in description.items()}, metadata)

    def tensor(self, name: str, device: torch.device | str = "cpu") -> torch.Tensor:
        """One tensor, read with safetensors (no pickle)."""
        from safetensors import safe_open

        shard = self.weight_map.get(name)
        if shard is None:
            raise KeyError(f"tensor {name!r} is not in the checkpoint")
        handle = self._handles.get(shard)
        if handle is None:
            handle = safe_open(str(self.path / shard), framework="pt", device="cpu")
            self._handles[shard] = handle
        return handle.get_tensor(name).to(device)

    def quant_type(self, component: str) -> str:
        return self.description.get(f"{component}.weight", FLOAT_TYPE)

    def static_linear(self, components: Sequence[str], device: torch.device | str) -> torch.nn.Module:
        """A processed W8A8HIF8_STATIC Linear from one or more fused components.

        Weights and channel scales are concatenated along N in the given order;
        every component must carry the same input scale.
        """
        if not components:
            raise ValueError("static_linear needs at least one component")
        weights, scales, input_scale = [], [], None
        for comp in components:
            if self.quant_type(comp) != STATIC_QUANT_TYPE:
                raise ValueError(f"{comp}.weight is {self.quant_type(comp)}, expected {STATIC_QUANT_TYPE}")
            w = self.tensor(f"{comp}.weight")
            ws = self.tensor(f"{comp}.weight_scale")
            xs = self.tensor(f"{comp}.input_scale")
            if w.dtype != torch.uint8 or w.dim() != 2:
                raise TypeError(f"{comp}.weight must be U8 [N, K], got {w.dtype} {tuple(w.shape)}")
            if ws.dtype != torch.float32 or ws.numel() != w.shape[0]:
                raise TypeError(f"{comp}.weight_scale must be F32 [N, 1] with N={w.shape[0]}")
            if xs.dtype != torch.float32 or xs.numel() != 1:
                raise TypeError(f"{comp}.input_scale must be F32 [1]")
            if input_scale is None:
                input_scale = xs.reshape(1)
            elif not torch.equal(input_scale, xs.reshape(1)):
                raise ValueError(f"fused components {list(components)} have different input scales")
            weights.append(w)
            scales.append(ws.reshape(-1, 1))
        if len({w.shape[1] for w in weights}) != 1:
            raise ValueError(f"fused components {list(components)} have different K")
        layer = torch.nn.Module()
        layer.weight = torch.nn.Parameter(torch.cat(weights).to(device), requires_grad=False)
        layer.weight_scale = torch.nn.Parameter(torch.cat(scales).to(device), requires_grad=False)
        layer.input_scale = torch.nn.Parameter(input_scale.to(device), requires_grad=False)
        method = scheme.W8A8HiFloat8StaticLinearMethod()
        method.process_weights_after_loading(layer)
        layer.quant_method = method
        return layer

    def embedding(self, component: str, device: torch.device | str) -> torch.nn.Module:
        """The W8A8HIF8_SOFT token embedding (rows + per-row scales)."""
        if self.quant_type(component) != SOFT_QUANT_TYPE:
            raise ValueError(f"{component}.weight is {self.quant_type(component)}, expected {SOFT_QUANT_TYPE}")
        layer = torch.nn.Module()
        layer.weight = torch.nn.Parameter(self.tensor(f"{component}.weight", device), requires_grad=False)
        layer.weight_scale = torch.nn.Parameter(self.tensor(f"{component}.weight_scale", device),
                                                requires_grad=False)
        method = scheme.W8A8HiFloat8SoftEmbeddingMethod()
        method.process_weights_after_loading(layer)
        layer.quant_method = method
        return layer

    def kv_scales(self, layer_index: int, device: torch.device | str) -> tuple[torch.Tensor, torch.Tensor]:
        """float32 per-head K and V scales of one full-attention layer."""
        scales = load_static_kv_scales(self.path)
        if scales is None or layer_index not in scales:
            raise KeyError(f"no static KV scales for layer {layer_index}")
        key, value = scales[layer_index]
        return (torch.tensor(key, dtype=torch.float32, device=device),
                torch.tensor(value, dtype=torch.float32, device=device))


def _weight_map(directory: Path) -> dict[str, str]:
    """Tensor -> shard file, from the safetensors index or the single file (exporter.py:330-345)."""
    index = directory / "model.safetensors.index.json"
    if index.exists():
        data = json.loads(index.read_text(encoding="utf-8"))
        weight_map = data.get("weight_map")
        if not isinstance(weight_map, dict) or not weight_map:
            raise ValueError(f"invalid safetensors index: {index}")
        return {str(k): str(v) for k, v in weight_map.items()}
    single = directory / "model.safetensors"
    if single.exists():
        from safetensors import safe_open

        with safe_open(str(single), framework="pt", device="cpu") as handle:
            return {name: single.name for name in handle.keys()}
    raise FileNotFoundError(f"no model.safetensors or model.safetensors.index.json in {directory}")


__all__ = [
    "FLOAT_TYPE",
    "Hif8Checkpoint",
    "KV_MODE",
    "METADATA_FILENAME",
    "QUANT_DESCRIPTION_FILENAME",
    "SOFT_QUANT_TYPE",
    "STATIC_QUANT_TYPE",
    "load_static_kv_scales",
]
