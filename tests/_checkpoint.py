"""A tiny synthetic exported checkpoint in the reference's on-disk format
(docs/checkpoint-format.md:5-57): two safetensors shards behind an index,
fused q/k/v and gate/up components sharing an input scale, a SOFT token
embedding, a FLOAT norm, the quant description and the KV metadata."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch
from safetensors.torch import save_file

from _data import hif8_weight

HIDDEN = 256
VOCAB = 96
QKV = {"q_proj": 128, "k_proj": 64, "v_proj": 64}
GATE_UP = {"gate_proj": 192, "up_proj": 192}
ATTN = "model.layers.3.self_attn"
MLP = "model.layers.3.mlp"
EMBED = "model.embed_tokens"
KV_SCALES = {"key_scales": [0.125, 0.0625], "value_scales": [0.25, 0.5]}


def write_checkpoint(root: Path, *, single_file: bool = False, qkv_input_scales=(0.01, 0.01, 0.01),
                     metadata: dict | None = None) -> dict[str, torch.Tensor]:
    tensors: dict[str, torch.Tensor] = {}
    description: dict[str, str] = {}
    seed = 7
    for prefix, comps, scales in ((ATTN, QKV, qkv_input_scales), (MLP, GATE_UP, (0.02, 0.02))):
        for (name, n), xs in zip(comps.items(), scales):
            w, ws = hif8_weight(n, HIDDEN, seed=seed)
            seed += 1
            tensors[f"{prefix}.{name}.weight"] = torch.from_numpy(w)
            tensors[f"{prefix}.{name}.weight_scale"] = torch.from_numpy(ws.astype(np.float32)).reshape(n, 1)
            tensors[f"{prefix}.{name}.input_scale"] = torch.tensor([xs], dtype=torch.float32)
            description[f"{prefix}.{name}.weight"] = "W8A8HIF8_STATIC"
            description[f"{prefix}.{name}.weight_scale"] = "W8A8HIF8_STATIC"
            description[f"{prefix}.{name}.input_scale"] = "W8A8HIF8_STATIC"
    ew, es = hif8_weight(VOCAB, HIDDEN, seed=99)
    tensors[f"{EMBED}.weight"] = torch.from_numpy(ew)
    tensors[f"{EMBED}.weight_scale"] = torch.from_numpy(es.astype(np.float32)).reshape(VOCAB, 1)
    description[f"{EMBED}.weight"] = "W8A8HIF8_SOFT"
    description[f"{EMBED}.weight_scale"] = "W8A8HIF8_SOFT"
    tensors["model.norm.weight"] = torch.ones(HIDDEN, dtype=torch.bfloat16)
    description["model.norm.weight"] = "FLOAT"

    root.mkdir(parents=True, exist_ok=True)
    if single_file:
        save_file(tensors, str(root / "model.safetensors"))
    else:
        names = sorted(tensors)
        half = len(names) // 2
        shards = {"model-00001-of-00002.safetensors": names[:half],
                  "model-00002-of-00002.safetensors": names[half:]}
        weight_map = {}
        for shard, members in shards.items():
            save_file({k: tensors[k] for k in members}, str(root / shard))
            weight_map.update({k: shard for k in members})
        (root / "model.safetensors.index.json").write_text(
            json.dumps({"metadata": {}, "weight_map": weight_map}), encoding="utf-8")
    (root / "quant_model_description.json").write_text(json.dumps(description), encoding="utf-8")
    if metadata is None:
        metadata = {"format": "W8A8HIF8_STATIC",
                    "kv_cache": {"mode": "static_per_layer_per_head", "layers": {"3": dict(KV_SCALES)}}}
    (root / "hif8_metadata.json").write_text(json.dumps(metadata), encoding="utf-8")
    return tensors
