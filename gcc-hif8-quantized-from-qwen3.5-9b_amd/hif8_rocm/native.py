"""Python operator API for the HiF8 HIP kernels.

Mirrors the reference's ``vllm_ascend_hif8.native`` (native.py:28-304): the
same function names, argument meaning, validation messages and exception
types.  Operators are reached through ``torch.ops.vllm_ascend_hif8.*`` (the
extension registers the reference's schemas) or, failing that, the extension
module's functions.  There is no fallback: a missing extension raises
:class:`NativeExtensionUnavailable`.
"""

from __future__ import annotations

import importlib
import os
from types import ModuleType
from typing import TYPE_CHECKING

if TYPE_CHECKING:
    import torch

_EXTENSION_MODULE = "hif8_rocm._C"
_REQUIRED_SYMBOLS = (
    "hif8_dynamic_quant",
    "hif8_static_quant",
    "soft_hif8_gemv",
    "soft_hif8_gemm",
)
_extension: ModuleType | None = None
_load_error: BaseException | None = None

# Routing thresholds of the reference's soft_linear (native.py:22-25).  Both
# operators reach the same HBM-streaming GEMV kernel for M <= 4 here.
_SOFT_HIF8_GEMV_MAX_OUTPUT_COLUMNS = 1_536
_SOFT_HIF8_GEMV_MAX_INPUT_COLUMNS = 8_192
_DISABLE_GEMV_ENV = "HIF8_DISABLE_GEMV"


class NativeExtensionUnavailable(RuntimeError):
    """Raised when the HiF8 HIP operators cannot be loaded."""


def load_extension() -> ModuleType:
    """Import ``hif8_rocm._C`` once and hand it back (reference loader: native.py:32-50).

    The outcome is memoised either way: after a failed import every later
    call raises :class:`NativeExtensionUnavailable` again, chained to the
    original error, without retrying the import.
    """
    global _extension, _load_error
    if _extension is not None:
        return _extension
    if _load_error is not None:
        raise NativeExtensionUnavailable(_unavailable_text()) from _load_error
    try:
        module = importlib.import_module(_EXTENSION_MODULE)
        absent = [name for name in _REQUIRED_SYMBOLS if not callable(getattr(module, name, None))]
        if absent:
            raise ImportError("hif8_rocm._C lacks the operator entry points " + ", ".join(absent))
    except BaseException as exc:  # noqa: BLE001 - memoised, surfaced as NativeExtensionUnavailable
        _load_error = exc
        raise NativeExtensionUnavailable(_unavailable_text()) from exc
    _extension = module
    return module


def _unavailable_text() -> str:
    cause = "" if _load_error is None else f" ({_load_error})"
    return (
        f"the HiF8 HIP extension could not be loaded{cause}; compile it with __graft_entry__.build() "
        "or python -m hif8_rocm._build. These operators run only on the HIP kernels (there is "
        "no decoded-weight or floating-point fallback)."
    )


def is_available() -> bool:
    """True when the extension imports and exports every required operator."""
    try:
        load_extension()
    except NativeExtensionUnavailable:
        return False
    return True


def reset_extension_cache() -> None:
    """Forget the memoised import result, so that the next call imports again."""
    global _extension, _load_error
    _extension = None
    _load_error = None


def _operator(name: str, extension: ModuleType):
    import torch

    namespace = torch.ops.vllm_ascend_hif8
    try:
        op = getattr(namespace, name)
    except (AttributeError, RuntimeError):
        op = None
    if op is None:
        op = getattr(extension, name, None)
    if not callable(op):
        raise NativeExtensionUnavailable(f"the native extension has no {name} operator; rebuild it")
    return op


def dynamic_quant(x: "torch.Tensor") -> tuple["torch.Tensor", "torch.Tensor"]:
    """Quantize BF16/FP16 activations into U8 HiFloat8 with FP32 token scales (native.py:77-87).

    Row r's scale is max(finite amax of the row, 1e-12); the row scales come
    back contiguous ``[rows]``.
    """
    extension = load_extension()
    x = _as_native_operand(x)
    data, scale = _operator("hif8_dynamic_quant", extension)(x)
    _validate_quantized_activation(x, data, scale, operation="hif8_dynamic_quant")
    return data, scale


def static_quant(x: "torch.Tensor", fixed_scale: "torch.Tensor") -> tuple["torch.Tensor", "torch.Tensor"]:
    """Quantize with fixed FP32 scale(s), without an activation reduction (native.py:90-124).

    One scale is used for every row of a Linear activation.  For KV tensors,
    flatten ``[tokens, heads, dim]`` into ``[tokens * heads, dim]`` and pass one
    scale per head; row r uses ``fixed_scale[r % S]``.
    """
    import torch

    if x.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"static HiFloat8 quant requires FP16/BF16 input, got {x.dtype}")
    if x.ndim < 1:
        raise ValueError("static HiFloat8 quant requires at least one dimension")
    if fixed_scale.dtype != torch.float32 or fixed_scale.ndim != 1:
        raise TypeError("fixed_scale must be a 1D torch.float32 tensor")
    rows = x.numel() // x.shape[-1]
    if fixed_scale.numel() <= 0 or rows % fixed_scale.numel():
        raise ValueError(f"fixed_scale count {fixed_scale.numel()} must divide {rows} activation rows")
    if fixed_scale.device != x.device:
        raise ValueError(f"fixed_scale must be on {x.device}, got {fixed_scale.device}")
    x = _as_native_operand(x)
    fixed_scale = _as_native_operand(fixed_scale)
    extension = load_extension()
    data, scale = _operator("hif8_static_quant", extension)(x, fixed_scale)
    _validate_quantized_activation(x, data, scale, operation="hif8_static_quant")
    return data, scale


def scaled_decode(data: "torch.Tensor", scale: "torch.Tensor") -> "torch.Tensor":
    """Decode U8 HiFloat8 rows with FP32 scales into BF16 (native.py:127-145)."""
    import torch

    if data.dtype != torch.uint8:
        raise TypeError(f"scaled_decode requires uint8 data, got {data.dtype}")
    if scale.dtype != torch.float32:
        raise TypeError(f"scaled_decode requires float32 scale, got {scale.dtype}")
    if data.ndim != 2:
        raise ValueError(f"scaled_decode requires 2D data, got shape {data.shape}")
    extension = load_extension()
    data = _as_native_operand(data)
    scale = _as_native_operand(scale.reshape(-1))
    return _operator("hif8_scaled_decode", extension)(data, scale)


def embedding_lookup(
    weight: "torch.Tensor",
    weight_scale: "torch.Tensor",
    input_ids: "torch.Tensor",
    *,
    validate: bool = True,
) -> "torch.Tensor":
    """Gather and decode token-embedding rows into BF16 (scheme.py:121-131).

    ``out[..., :] = bf16(decode(weight[id]) * bf16(weight_scale[id]))`` with the
    shape ``[*input_ids.shape, dim]``.  With ``validate`` an id outside the
    vocabulary raises IndexError (one host synchronisation, as index_select
    would); without it such rows are zeros.
    """
    import torch

    if weight.dtype != torch.uint8 or weight.ndim != 2:
        raise TypeError("embedding weight must be a 2-D torch.uint8 tensor")
    if input_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"input_ids must be int32 or int64, got {input_ids.dtype}")
    extension = load_extension()
    ids = _as_native_operand(input_ids.to(weight.device))
    scale = _as_native_operand(weight_scale.reshape(-1).to(torch.float32))
    invalid = torch.zeros(1, dtype=torch.int32, device=weight.device) if validate else None
    out = _operator("hif8_embedding_lookup", extension)(ids, _as_native_operand(weight), scale, invalid)
    if validate and int(invalid.item()):
        raise IndexError("embedding input_ids reference rows outside the vocabulary")
    return out


def _as_native_operand(tensor: "torch.Tensor") -> "torch.Tensor":
    """Return a contiguous, zero-offset tensor (native.py:148-157)."""
    if tensor.is_contiguous() and tensor.storage_offset() == 0:
        return tensor
    return tensor.contiguous().clone()


def soft_linear(
    activation: "torch.Tensor",
    weight: "torch.Tensor",
    activation_scale: "torch.Tensor",
    weight_scale: "torch.Tensor",
    bias: "torch.Tensor | None" = None,
    *,
    output_dtype: "torch.dtype",
) -> "torch.Tensor":
    """Dispatch physical U8 operands to the GEMV or GEMM operator (native.py:160-201)."""
    import torch

    if activation.dtype != torch.uint8 or weight.dtype != torch.uint8:
        raise TypeError("soft HiFloat8 linear requires uint8 activation and weight tensors")
    if activation.ndim < 2 or weight.ndim != 2:
        raise ValueError("activation must be at least 2D and weight must be 2D")
    if activation.shape[-1] != weight.shape[-1]:
        raise ValueError(
            f"incompatible K dimensions: activation={activation.shape[-1]}, weight={weight.shape[-1]}"
        )
    if activation_scale.dtype != torch.float32 or weight_scale.dtype != torch.float32:
        raise TypeError("soft HiFloat8 linear requires float32 activation and weight scales")

    extension = load_extension()
    flattened = _as_native_operand(activation.reshape(-1, activation.shape[-1]))
    token_scale = _as_native_operand(activation_scale.reshape(-1))
    channel_scale = _as_native_operand(weight_scale.reshape(-1))
    if token_scale.numel() != flattened.shape[0]:
        raise ValueError("activation_scale must contain one value per token row")
    if channel_scale.numel() != weight.shape[0]:
        raise ValueError("weight_scale must contain one value per output channel")

    use_gemv = (
        os.environ.get(_DISABLE_GEMV_ENV) != "1"
        and flattened.shape[0] == 1
        and weight.shape[0] <= _SOFT_HIF8_GEMV_MAX_OUTPUT_COLUMNS
        and flattened.shape[1] <= _SOFT_HIF8_GEMV_MAX_INPUT_COLUMNS
    )
    operator = _operator("soft_hif8_gemv" if use_gemv else "soft_hif8_gemm", extension)
    output = operator(flattened, weight, token_scale, channel_scale, bias, output_dtype)
    return output.reshape(*activation.shape[:-1], weight.shape[0])


def decode_weight(weight: "torch.Tensor") -> "torch.Tensor":
    """HiF8 codes -> bf16 (exact; no counterpart in the reference): the weight
    that ``soft_linear_decoded_weight`` reads, 2 bytes per element."""
    import torch

    if weight.dtype != torch.uint8:
        raise TypeError(f"decode_weight requires a uint8 tensor, got {weight.dtype}")
    if weight.numel() % 16:
        raise ValueError(f"decode_weight requires a multiple of 16 elements, got {weight.numel()}")
    extension = load_extension()
    return _operator("hif8_decode_bf16", extension)(_as_native_operand(weight))


def soft_linear_decoded_weight(
    activation: "torch.Tensor",
    weight_bf16: "torch.Tensor",
    activation_scale: "torch.Tensor",
    weight_scale: "torch.Tensor",
    bias: "torch.Tensor | None" = None,
    *,
    output_dtype: "torch.dtype",
) -> "torch.Tensor":
    """``soft_linear`` for prefill with the weight kept decoded (``decode_weight``):
    the same results (FP32 summation order aside) with no per-call weight
    decode; requires K % 64 == 0.  No counterpart in the reference."""
    import torch

    if activation.dtype != torch.uint8 or weight_bf16.dtype != torch.bfloat16:
        raise TypeError("soft_linear_decoded_weight requires uint8 activation codes and a bfloat16 weight")
    if activation.ndim < 2 or weight_bf16.ndim != 2:
        raise ValueError("activation must be at least 2D and weight must be 2D")
    if activation.shape[-1] != weight_bf16.shape[-1]:
        raise ValueError(
            f"incompatible K dimensions: activation={activation.shape[-1]}, weight={weight_bf16.shape[-1]}"
        )
    if activation_scale.dtype != torch.float32 or weight_scale.dtype != torch.float32:
        raise TypeError("soft HiFloat8 linear requires float32 activation and weight scales")
    extension = load_extension()
    flattened = _as_native_operand(activation.reshape(-1, activation.shape[-1]))
    token_scale = _as_native_operand(activation_scale.reshape(-1))
    channel_scale = _as_native_operand(weight_scale.reshape(-1))
    if token_scale.numel() != flattened.shape[0]:
        raise ValueError("activation_scale must contain one value per token row")
    if channel_scale.numel() != weight_bf16.shape[0]:
        raise ValueError("weight_scale must contain one value per output channel")
    operator = _operator("soft_hif8_gemm_decoded_weight", extension)
    output = operator(flattened, _as_native_operand(weight_bf16), token_scale, channel_scale, bias, output_dtype)
    return output.reshape(*activation.shape[:-1], weight_bf16.shape[0])


def soft_fused_linear(
    x: "torch.Tensor",
    weight: "torch.Tensor",
    weight_scale: "torch.Tensor",
    bias: "torch.Tensor | None" = None,
    *,
    output_dtype: "torch.dtype",
) -> "torch.Tensor":
    """Fused dynamic activation quant/decode with U8-weight GEMV, M <= 2 (native.py:205-238)."""
    import torch

    if x.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"fused soft HiFP8 linear requires FP16/BF16 activation, got {x.dtype}")
    if weight.dtype != torch.uint8 or weight.ndim != 2:
        raise TypeError("fused soft HiFP8 linear requires a 2D uint8 weight tensor")
    if x.ndim < 2 or x.shape[-1] != weight.shape[-1]:
        raise ValueError("activation and weight must have compatible final K dimensions")
    if weight_scale.dtype != torch.float32 or weight_scale.numel() != weight.shape[0]:
        raise TypeError("fused soft HiFP8 linear requires one float32 scale per output channel")

    flattened = _as_native_operand(x.reshape(-1, x.shape[-1]))
    if flattened.shape[0] > 2:
        raise ValueError("fused soft HiFP8 linear supports M <= 2")
    channel_scale = _as_native_operand(weight_scale.reshape(-1))
    extension = load_extension()
    operator = _operator("soft_hif8_fused_gemm", extension)
    output = operator(flattened, weight, channel_scale, bias, output_dtype)
    return output.reshape(*x.shape[:-1], weight.shape[0])


def soft_static_fused_linear(
    x: "torch.Tensor",
    weight: "torch.Tensor",
    fixed_scale: "torch.Tensor",
    weight_scale: "torch.Tensor",
    bias: "torch.Tensor | None" = None,
    *,
    output_dtype: "torch.dtype",
) -> "torch.Tensor":
    """Fused fixed-scale activation encode with U8-weight GEMV, M <= 4 (native.py:241-284)."""
    import torch

    if x.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError(f"static fused soft HiFP8 linear requires FP16/BF16 activation, got {x.dtype}")
    if weight.dtype != torch.uint8 or weight.ndim != 2:
        raise TypeError("static fused soft HiFP8 linear requires a 2D uint8 weight tensor")
    if x.ndim < 2 or x.shape[-1] != weight.shape[-1]:
        raise ValueError("activation and weight must have compatible final K dimensions")
    if fixed_scale.dtype != torch.float32 or fixed_scale.ndim != 1 or fixed_scale.numel() != 1:
        raise TypeError("static fused soft HiFP8 linear requires one float32 activation scale")
    if weight_scale.dtype != torch.float32 or weight_scale.numel() != weight.shape[0]:
        raise TypeError("static fused soft HiFP8 linear requires one float32 scale per output channel")
    if fixed_scale.device != x.device or weight_scale.device != x.device or weight.device != x.device:
        raise ValueError("activation, weight, fixed_scale, and weight_scale must be on the same device")

    flattened = _as_native_operand(x.reshape(-1, x.shape[-1]))
    fixed = _as_native_operand(fixed_scale.reshape(-1))
    channel_scale = _as_native_operand(weight_scale.reshape(-1))
    extension = load_extension()
    operator = _operator("soft_hif8_static_fused_gemm", extension)
    output = operator(flattened, weight, fixed, channel_scale, bias, output_dtype)
    return output.reshape(*x.shape[:-1], weight.shape[0])


def _validate_quantized_activation(source, data, scale, *, operation: str) -> None:
    """Post-conditions on a quantizer's outputs (native.py:287-304)."""
    import torch

    if data.dtype != torch.uint8:
        raise RuntimeError(f"{operation} returned {data.dtype}, expected torch.uint8")
    if data.shape != source.shape:
        raise RuntimeError(f"{operation} changed activation shape from {source.shape} to {data.shape}")
    if scale.dtype != torch.float32:
        raise RuntimeError(f"{operation} returned {scale.dtype} scale, expected torch.float32")
    expected_rows = source.numel() // source.shape[-1]
    if scale.numel() != expected_rows:
        raise RuntimeError(f"{operation} returned {scale.numel()} scales for {expected_rows} activation rows")
