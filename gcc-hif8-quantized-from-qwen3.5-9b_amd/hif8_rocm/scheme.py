"""Static W8A8 HiFloat8 linear method (the caller of the quant + GEMM path).

Mirrors ``AscendW8A8HiFloat8StaticLinearMethod`` (scheme.py:134-211) and its
weight processing (scheme.py:59-91) without the vLLM-Ascend registry: a layer
holds ``weight`` uint8 [N, K], ``weight_scale`` float32 [N, 1] and
``input_scale`` float32 [1]; ``apply`` statically quantises the activation and
runs the soft HiF8 linear.

The reference routes the fused static-quant GEMV only when
``HIF8_STATIC_FUSED_GENERATION=1``, M <= 4 and K < 1024 (scheme.py:181-189),
because on its hardware the fused kernel pays a global barrier.  The MI355X
fused kernels have none (every block encodes its own activation chunk) and
their outputs equal quant -> GEMM bit for bit.  Measured on MI355X in HIP
graphs, the separate quant launch costs 2-4 us of launch and cold-cache
latency, so decode-sized inputs go through the fused op by default: up to
``HIF8_STATIC_FUSED_ROWS`` token rows (default 4).  The op itself picks one
launch or quant + GEMV per shape: one row runs the one-row fused kernel (q
6.8 vs 9.0 us, k/v 5.0 vs 7.6, o 6.8 vs 9.0, gate_up 20.6 vs 21.3, down 13.6
vs 14.1);
four rows with K <= 4096 and N <= 2048 run the MFMA-4 GEMV's fused kind (k/v
8.2 vs 8.5 us; with more blocks the per-block re-encode of the rows costs
more than the quant launch); other shapes run quant + GEMV.
``HIF8_STATIC_FUSED_SINGLE_ROW=0`` or ``HIF8_STATIC_FUSED_ROWS=0`` restores
the reference's routing (static_quant -> soft_linear unless
``HIF8_STATIC_FUSED_GENERATION=1``, M <= 4, K < 1024, scheme.py:183-190);
``HIF8_STATIC_FUSED_ROWS=1`` fuses one row only.  The routing changes which
kernels run, not the outputs (equal bit for bit).

``HIF8_PREFILL_BF16_WEIGHTS=1`` (read in ``process_weights_after_loading``)
keeps each weight decoded to bf16 beside its codes (2 bytes per element;
HBM is 288 GB per MI355X) and runs GEMMs of more than four rows on it,
without the per-call weight decode; results equal the code path's up to
FP32 summation order.
"""

from __future__ import annotations

import math
import os
from typing import Any

import torch

from . import native

STATIC_QUANT_TYPE = "W8A8HIF8_STATIC"
_COMPUTE_BACKEND_ENV = "HIF8_COMPUTE_BACKEND"
_SOFT_HIF8_BACKEND = "soft_hif8"
_STATIC_FUSED_GENERATION_ENV = "HIF8_STATIC_FUSED_GENERATION"
_STATIC_SCALE_FACTOR_ENV = "HIF8_STATIC_SCALE_FACTOR"
# MI355X routing of decode-sized inputs through the fused op (see the module
# text): "0" in either variable restores the reference's routing.
_STATIC_FUSED_SINGLE_ROW_ENV = "HIF8_STATIC_FUSED_SINGLE_ROW"
_STATIC_FUSED_ROWS_ENV = "HIF8_STATIC_FUSED_ROWS"
# MI355X opt-in: keep each static weight decoded to bf16 for prefill GEMMs.
_PREFILL_BF16_WEIGHTS_ENV = "HIF8_PREFILL_BF16_WEIGHTS"


def _fused_rows() -> int:
    """Token rows up to which apply() routes through the fused op (0..4)."""
    if os.environ.get(_STATIC_FUSED_SINGLE_ROW_ENV, "1") == "0":
        return 0
    raw = os.environ.get(_STATIC_FUSED_ROWS_ENV)
    if raw is None or raw == "":
        return 4
    try:
        rows = int(raw)
    except ValueError as exc:
        raise ValueError(f"{_STATIC_FUSED_ROWS_ENV} must be an integer, got {raw!r}") from exc
    return max(0, min(rows, 4))


def _static_scale_factor() -> float:
    """Optional constant multiplier for calibrated static scales (scheme.py:26-40)."""
    raw = os.environ.get(_STATIC_SCALE_FACTOR_ENV)
    if raw is None or raw == "":
        return 1.0
    try:
        value = float(raw)
    except ValueError as exc:
        raise ValueError(f"{_STATIC_SCALE_FACTOR_ENV} must be a positive finite float") from exc
    if not math.isfinite(value) or value <= 0.0:
        raise ValueError(f"{_STATIC_SCALE_FACTOR_ENV} must be a positive finite float")
    return value


class W8A8HiFloat8StaticLinearMethod:
    """Calibrated per-tensor A8 and per-channel W8 HiFloat8 Linear (scheme.py:134-211)."""

    quant_type = STATIC_QUANT_TYPE
    supports_tp_weight_switch = False

    def get_weight(self, input_size: int, output_size: int, params_dtype: torch.dtype) -> dict[str, Any]:
        return {"weight": torch.empty(output_size, input_size, dtype=torch.uint8)}

    def get_perchannel_param(self, output_size: int, params_dtype: torch.dtype) -> dict[str, Any]:
        return {"weight_scale": torch.empty(output_size, 1, dtype=torch.float32)}

    def get_pertensor_param(self, params_dtype: torch.dtype, **kwargs: Any) -> dict[str, Any]:
        del params_dtype, kwargs
        return {"input_scale": torch.empty(1, dtype=torch.float32)}

    def _process_hif8_weights(self, layer: torch.nn.Module) -> None:
        """scheme.py:59-91 (the bf16 embedding LUT is not part of this path)."""
        if layer.weight.dtype != torch.uint8:
            raise TypeError(f"{self.quant_type} checkpoint weight must be torch.uint8, got {layer.weight.dtype}")
        if layer.weight_scale.dtype != torch.float32:
            layer.weight_scale.data = layer.weight_scale.data.to(torch.float32)
        layer.weight.data = layer.weight.data.contiguous()
        layer.weight_scale.data = layer.weight_scale.data.reshape(-1).contiguous()
        backend = os.environ.get(_COMPUTE_BACKEND_ENV, _SOFT_HIF8_BACKEND)
        if backend != _SOFT_HIF8_BACKEND:
            raise ValueError(
                f"unsupported {_COMPUTE_BACKEND_ENV}={backend!r}; only '{_SOFT_HIF8_BACKEND}' is supported"
            )
        layer._hif8_compute_backend = backend

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        """Validate and normalise the checkpoint tensors (scheme.py:157-172)."""
        if not hasattr(layer, "input_scale"):
            raise ValueError(f"{STATIC_QUANT_TYPE} checkpoint is missing input_scale")
        scale = layer.input_scale.data.to(dtype=torch.float32).reshape(-1)
        if scale.numel() != 1:
            raise ValueError(
                f"{STATIC_QUANT_TYPE} requires one input_scale value, got shape {tuple(layer.input_scale.shape)}"
            )
        if not bool(torch.isfinite(scale).all()) or not bool((scale > 0).all()):
            raise ValueError(f"{STATIC_QUANT_TYPE} input_scale must be finite and greater than zero")
        layer.input_scale.data = scale.contiguous()
        self._process_hif8_weights(layer)
        # MI355X opt-in: keep the weight decoded to bf16 as well (2 bytes per
        # element) so prefill GEMMs skip the per-call weight decode.
        layer._hif8_weight_bf16 = None
        if (
            os.environ.get(_PREFILL_BF16_WEIGHTS_ENV) == "1"
            and layer.weight.is_cuda
            and layer.weight.shape[-1] % 64 == 0
        ):
            layer._hif8_weight_bf16 = native.decode_weight(layer.weight.data)

    def apply(
        self,
        layer: torch.nn.Module,
        x: torch.Tensor,
        bias: torch.Tensor | None = None,
        tp_rank: int | None = 0,
    ) -> torch.Tensor:
        """static_quant -> soft_linear, or the fused kernel (scheme.py:174-211).

        Fused when the reference would fuse (``HIF8_STATIC_FUSED_GENERATION=1``,
        M <= 4, K < 1024) and for up to ``HIF8_STATIC_FUSED_ROWS`` token rows
        (default 4; 0 or ``HIF8_STATIC_FUSED_SINGLE_ROW=0`` turns it off); the
        routes give equal outputs."""
        del tp_rank
        token_rows = x.numel() // x.shape[-1]
        k = x.shape[-1]
        use_fused = (
            token_rows <= 4 and os.environ.get(_STATIC_FUSED_GENERATION_ENV) == "1" and k < 1024
        ) or token_rows <= _fused_rows()
        scale_factor = _static_scale_factor()
        fixed_scale = layer.input_scale
        if scale_factor != 1.0:
            fixed_scale = fixed_scale * scale_factor
        if use_fused:
            return native.soft_static_fused_linear(
                x, layer.weight, fixed_scale, layer.weight_scale, bias, output_dtype=x.dtype
            )
        activation, row_scale = native.static_quant(x, fixed_scale)
        decoded = getattr(layer, "_hif8_weight_bf16", None)
        if decoded is not None and token_rows > 4:
            return native.soft_linear_decoded_weight(
                activation, decoded, row_scale, layer.weight_scale, bias, output_dtype=x.dtype
            )
        return native.soft_linear(
            activation, layer.weight, row_scale, layer.weight_scale, bias, output_dtype=x.dtype
        )


SOFT_QUANT_TYPE = "W8A8HIF8_SOFT"
_SOFT_FUSED_GENERATION_ENV = "HIF8_SOFT_FUSED_GENERATION"


class W8A8HiFloat8SoftLinearMethod:
    """Dynamic per-token A8 and per-channel W8 HiFloat8 (the W8A8HIF8_SOFT type, scheme.py:43-131).

    The legacy scheme: each activation row is quantised with its own scale
    (``hif8_dynamic_quant``) before the soft GEMM; with
    ``HIF8_SOFT_FUSED_GENERATION=1`` and at most two token rows the fused
    dynamic-scale GEMV runs instead.  Exported checkpoints also load their
    token embedding through this type; :meth:`embedding` gathers and decodes
    only the requested rows.
    """

    quant_type = SOFT_QUANT_TYPE
    supports_tp_weight_switch = False

    def get_weight(self, input_size: int, output_size: int, params_dtype: torch.dtype) -> dict[str, Any]:
        return {"weight": torch.empty(output_size, input_size, dtype=torch.uint8)}

    def get_perchannel_param(self, output_size: int, params_dtype: torch.dtype) -> dict[str, Any]:
        return {"weight_scale": torch.empty(output_size, 1, dtype=torch.float32)}

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        """scheme.py:59-91 (the decode table lives in the kernels, not in a buffer)."""
        if layer.weight.dtype != torch.uint8:
            raise TypeError(f"{self.quant_type} checkpoint weight must be torch.uint8, got {layer.weight.dtype}")
        if layer.weight_scale.dtype != torch.float32:
            layer.weight_scale.data = layer.weight_scale.data.to(torch.float32)
        layer.weight.data = layer.weight.data.contiguous()
        layer.weight_scale.data = layer.weight_scale.data.reshape(-1).contiguous()
        backend = os.environ.get(_COMPUTE_BACKEND_ENV, _SOFT_HIF8_BACKEND)
        if backend != _SOFT_HIF8_BACKEND:
            raise ValueError(
                f"unsupported {_COMPUTE_BACKEND_ENV}={backend!r}; only '{_SOFT_HIF8_BACKEND}' is supported"
            )
        layer._hif8_compute_backend = backend

    def apply(
        self,
        layer: torch.nn.Module,
        x: torch.Tensor,
        bias: torch.Tensor | None = None,
        tp_rank: int | None = 0,
    ) -> torch.Tensor:
        """dynamic_quant -> soft_linear, or the fused kernel for one or two rows (scheme.py:93-118)."""
        del tp_rank
        token_rows = x.numel() // x.shape[-1]
        if token_rows <= 2 and os.environ.get(_SOFT_FUSED_GENERATION_ENV) == "1":
            return native.soft_fused_linear(x, layer.weight, layer.weight_scale, bias, output_dtype=x.dtype)
        activation, activation_scale = native.dynamic_quant(x)
        return native.soft_linear(
            activation, layer.weight, activation_scale, layer.weight_scale, bias, output_dtype=x.dtype
        )

    def embedding(self, layer: torch.nn.Module, input_ids: torch.Tensor) -> torch.Tensor:
        """Gather and dequantize only the requested token embedding rows (scheme.py:121-131)."""
        return native.embedding_lookup(layer.weight, layer.weight_scale, input_ids)


# The token embedding of an exported checkpoint loads through the same type.
W8A8HiFloat8SoftEmbeddingMethod = W8A8HiFloat8SoftLinearMethod
