"""HiFloat8 paged KV cache: layout, the fused static write and decode attention.

Mirrors the reference's ``vllm_ascend_hif8.kv_cache`` layout API
(kv_cache.py:22-184) and replaces its adapter's write and attention sequences
(kv_runtime.py:1168-1339 and 1375-1563) with two native operators:

* :func:`write_kv_cache` - static quant with per-head checkpoint scales, row
  packing and slot scatter in one kernel (bytes identical to
  ``static_quant -> pack_kv_rows -> index_copy_``);
* :func:`paged_decode_attention` - one query token per request; the kernel reads
  only the pages in the block table and decodes them on chip, instead of
  gathering and materialising bf16 K/V for a fused-attention call.

K and V are separate uint8 tensors ``[num_blocks, block_size, num_kv_heads,
head_size + 4]``; a row is HiF8 codes followed by a little-endian FP32 scale.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

from . import native

HIF8_SCALE_BYTES = 4
HIF8_CACHE_DTYPE = "fp8_per_token_head"


@dataclass(frozen=True)
class Hif8KVCacheLayout:
    """Physical layout of one K/V cache pair (kv_cache.py:26-88)."""

    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_size: int
    head_size_v: int | None = None

    def __post_init__(self) -> None:
        head_size_v = self.head_size if self.head_size_v is None else self.head_size_v
        values = (self.num_blocks, self.block_size, self.num_kv_heads, self.head_size, head_size_v)
        if any(not isinstance(value, int) or value <= 0 for value in values):
            raise ValueError(f"HIF8 KV dimensions must be positive integers, got {values}")
        if self.head_size % HIF8_SCALE_BYTES:
            raise ValueError(
                "HIF8 KV head_size must be divisible by four so the inline FP32 "
                f"scale is aligned, got {self.head_size}"
            )
        if head_size_v % HIF8_SCALE_BYTES:
            raise ValueError(
                "HIF8 KV head_size_v must be divisible by four so the inline FP32 "
                f"scale is aligned, got {head_size_v}"
            )

    @property
    def resolved_head_size_v(self) -> int:
        return self.head_size if self.head_size_v is None else self.head_size_v

    @property
    def key_width(self) -> int:
        return self.head_size + HIF8_SCALE_BYTES

    @property
    def value_width(self) -> int:
        return self.resolved_head_size_v + HIF8_SCALE_BYTES

    @property
    def page_size_bytes(self) -> int:
        return self.block_size * self.num_kv_heads * (self.key_width + self.value_width)

    @property
    def key_page_size_bytes(self) -> int:
        return self.block_size * self.num_kv_heads * self.key_width

    @property
    def value_page_size_bytes(self) -> int:
        return self.block_size * self.num_kv_heads * self.value_width

    def key_shape(self) -> tuple[int, int, int, int]:
        return (self.num_blocks, self.block_size, self.num_kv_heads, self.key_width)

    def value_shape(self) -> tuple[int, int, int, int]:
        return (self.num_blocks, self.block_size, self.num_kv_heads, self.value_width)

    def allocate(self, device: torch.device | str) -> tuple[torch.Tensor, torch.Tensor]:
        """Zero-filled K and V caches of this layout on ``device``."""
        return (
            torch.zeros(self.key_shape(), dtype=torch.uint8, device=device),
            torch.zeros(self.value_shape(), dtype=torch.uint8, device=device),
        )


def pack_kv_rows(data: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Pack ``[T, H, D]`` codes and ``[T, H]`` FP32 scales into ``[T, H, D + 4]`` rows (kv_cache.py:151-170)."""
    if data.dtype != torch.uint8 or data.ndim != 3:
        raise TypeError("data must be a 3-D torch.uint8 tensor")
    if scale.dtype != torch.float32 or scale.shape != data.shape[:2]:
        raise TypeError("scale must be float32 with shape [tokens, heads]")
    if data.shape[-1] % HIF8_SCALE_BYTES:
        raise ValueError("head dimension must be divisible by four for inline scales")
    packed = torch.empty((*data.shape[:-1], data.shape[-1] + HIF8_SCALE_BYTES), dtype=torch.uint8,
                         device=data.device)
    packed[..., :-HIF8_SCALE_BYTES].copy_(data)
    packed[..., -HIF8_SCALE_BYTES:].copy_(
        scale.contiguous().view(torch.uint8).reshape(*scale.shape, HIF8_SCALE_BYTES))
    return packed


def unpack_kv_rows(packed: torch.Tensor, head_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Split ``[T, H, D + 4]`` rows into codes and FP32 scales (kv_cache.py:173-184)."""
    if packed.dtype != torch.uint8 or packed.ndim != 3:
        raise TypeError("packed must be a 3-D torch.uint8 tensor")
    expected = head_size + HIF8_SCALE_BYTES
    if packed.shape[-1] != expected:
        raise ValueError(f"packed last dimension must be {expected}, got {packed.shape[-1]}")
    data = packed[..., :head_size]
    scale = packed[..., head_size:].contiguous().view(torch.float32).reshape(*packed.shape[:2])
    return data, scale


def _check_caches(key_cache: torch.Tensor, value_cache: torch.Tensor) -> None:
    for name, cache in (("key_cache", key_cache), ("value_cache", value_cache)):
        if cache.dtype != torch.uint8 or cache.ndim != 4:
            raise TypeError(f"{name} must be a 4-D uint8 tensor")
        if not cache.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if key_cache.shape[:3] != value_cache.shape[:3]:
        raise ValueError("key_cache and value_cache must have the same blocks and heads")


def write_kv_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    key_scale: torch.Tensor,
    value_scale: torch.Tensor,
    *,
    num_actual_tokens: int | None = None,
    validate: bool = True,
) -> None:
    """Quantise ``key``/``value`` ``[T, Hkv, D]`` with per-head scales into the caches, in place.

    Static branch of ``_write_hif8_cache`` (kv_runtime.py:1222-1339): row (t, h)
    becomes ``static_encode(x / scale[h])`` plus the sidecar ``scale[h]`` at
    slot ``slot_mapping[t]``; negative slots are padding and are skipped.  With
    ``validate`` a slot beyond the cache raises IndexError before anything is
    written (one host synchronisation, as in the reference); without it such
    tokens are skipped on the device.
    """
    if key is None or value is None:
        raise ValueError("HIF8 KV cache update requires both key and value")
    _check_caches(key_cache, value_cache)
    if key.ndim != 3 or value.ndim != 3:
        raise ValueError(f"expected K/V [tokens, heads, dim], got {tuple(key.shape)} / {tuple(value.shape)}")
    if key.shape[-1] + HIF8_SCALE_BYTES != key_cache.shape[-1] or \
            value.shape[-1] + HIF8_SCALE_BYTES != value_cache.shape[-1]:
        raise ValueError(
            "HIF8 KV input dimensions do not match the cache rows: "
            f"K={key.shape[-1]}+4/{key_cache.shape[-1]}, V={value.shape[-1]}+4/{value_cache.shape[-1]}"
        )
    tokens = key.shape[0] if num_actual_tokens is None else int(num_actual_tokens)
    if tokens < 0 or tokens > key.shape[0] or tokens > value.shape[0]:
        raise ValueError(f"invalid num_actual_tokens={tokens} for K/V rows {key.shape[0]}/{value.shape[0]}")
    slots = slot_mapping[:tokens]
    if slots.dtype not in (torch.int32, torch.int64):
        slots = slots.to(torch.int64)
    slots = native._as_native_operand(slots.to(key_cache.device))
    if validate and tokens:
        capacity = key_cache.shape[0] * key_cache.shape[1]
        if bool((slots >= capacity).any()):
            raise IndexError("HIF8 KV slot mapping references an invalid block")
    extension = native.load_extension()
    native._operator("hif8_kv_cache_write", extension)(
        key[:tokens].contiguous(), value[:tokens].contiguous(), key_cache, value_cache, slots,
        key_scale.to(torch.float32).contiguous(), value_scale.to(torch.float32).contiguous(), None)


def paged_decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: Sequence[int] | torch.Tensor,
    *,
    scale: float,
    max_seq_len: int | None = None,
    validate: bool = True,
) -> torch.Tensor:
    """Decode attention over HiF8 pages: ``query`` ``[B, Hq, D]`` -> ``[B, Hq, Dv]``.

    One query token per request (the last position, so the causal mask admits
    every cached token); the contract is ``paged_attention_reference``
    (kv_cache.py:314-372) with ``query_lens`` all 1.  ``seq_lens`` may be a host
    sequence (as the reference's ``seq_lens_list``) or an int32 device tensor;
    with a tensor, pass ``max_seq_len`` to avoid a host synchronisation.
    ``validate`` checks the block ids that the lengths reach (kv_cache.py:247-249).
    """
    _check_caches(key_cache, value_cache)
    if query.ndim != 3:
        raise ValueError("query must have shape [tokens, num_heads, head_size]")
    batch = query.shape[0]
    if query.shape[1] % key_cache.shape[2]:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    if block_table.ndim != 2 or block_table.shape[0] < batch:
        raise ValueError("block_table must have shape [batch, max_blocks]")
    block_size = key_cache.shape[1]
    if isinstance(seq_lens, torch.Tensor):
        lens_dev = seq_lens.to(device=query.device, dtype=torch.int32).contiguous()
        if max_seq_len is None:
            max_seq_len = int(lens_dev.max().item()) if batch else 0
        lengths = None
    else:
        lengths = [int(v) for v in seq_lens]
        if len(lengths) != batch:
            raise ValueError("one sequence length is required per request")
        if any(v < 0 for v in lengths):
            raise ValueError("sequence lengths must be non-negative")
        lens_dev = torch.tensor(lengths, dtype=torch.int32).to(query.device)
        if max_seq_len is None:
            max_seq_len = max(lengths, default=0)
    if max_seq_len > block_table.shape[1] * block_size:
        raise ValueError("block_table has too few entries for a sequence length")
    table = block_table[:batch]
    if table.dtype not in (torch.int32, torch.int64):
        table = table.to(torch.int64)
    table = table.to(query.device).contiguous()
    if validate and batch and max_seq_len > 0:
        if bool((lens_dev > max_seq_len).any()):
            raise ValueError("max_seq_len is smaller than a sequence length")
        needed = (max_seq_len + block_size - 1) // block_size
        used = torch.arange(needed, device=query.device)[None, :] * block_size < lens_dev[:, None].to(torch.int64)
        ids = table[:, :needed].to(torch.int64)
        if bool(((ids < 0) | (ids >= key_cache.shape[0]))[used].any()):
            raise IndexError("block_table references a block outside the cache")
    extension = native.load_extension()
    return native._operator("hif8_paged_decode_attention", extension)(
        query.contiguous(), key_cache, value_cache, table, lens_dev, float(scale), int(max_seq_len))


def paged_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: Sequence[int] | torch.Tensor,
    *,
    scale: float,
    query_lens: Sequence[int] | None = None,
    query_start_loc: torch.Tensor | None = None,
    causal: bool = True,
    max_query_len: int | None = None,
    max_seq_len: int | None = None,
    validate: bool = True,
) -> torch.Tensor:
    """Attention over HiF8 pages for any number of query tokens per request.

    ``query`` is ``[T, Hq, D]`` in the TND layout; request b owns the next
    ``query_lens[b]`` rows, which are the last positions of its
    ``seq_lens[b]`` cached tokens (this step's cache write included), and with
    ``causal`` row i sees keys ``0 .. seq_lens[b] - query_lens[b] + i`` - the
    contract of ``paged_attention_reference`` with ``query_lens``
    (kv_cache.py:314-372) and of the reference's TND attention call
    (kv_runtime.py:1470-1563).  Returns ``[T, Hq, Dv]``.

    The request split comes from ``query_lens`` (host integers, as the
    reference's oracle takes them; rows must add up to T) or from
    ``query_start_loc`` (an int32 device tensor ``[B + 1]``, the cumulative
    form of the reference's ``actual_seq_lengths_q`` with a leading 0; pass
    ``max_query_len`` to avoid a host synchronisation, and ``validate=False``
    as well, since validation checks it against ``query_start_loc``).  One
    query row per request runs the decode kernel; otherwise the multi-token
    kernel.
    """
    _check_caches(key_cache, value_cache)
    if query.ndim != 3:
        raise ValueError("query must have shape [tokens, num_heads, head_size]")
    if query.shape[1] % key_cache.shape[2]:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    if (query_lens is None) == (query_start_loc is None):
        raise ValueError("pass exactly one of query_lens and query_start_loc")
    tokens = query.shape[0]
    if query_lens is not None:
        q_lengths = [int(v) for v in query_lens]
        if any(v < 0 for v in q_lengths) or sum(q_lengths) != tokens:
            raise ValueError("query_lens must describe every query row")
        batch = len(q_lengths)
        if not isinstance(seq_lens, torch.Tensor):
            lengths = [int(v) for v in seq_lens]
            if len(lengths) != batch:
                raise ValueError("one sequence length is required per request")
            for q_len, kv_len in zip(q_lengths, lengths):
                if q_len and kv_len < q_len:
                    raise ValueError(
                        "HIF8 post-update KV length cannot be shorter than its query "
                        f"length, got q={q_len}, kv={kv_len}")
        if batch == tokens and all(v == 1 for v in q_lengths):
            # The decode case: each row is its request's last position.
            return paged_decode_attention(query, key_cache, value_cache, block_table, seq_lens, scale=scale,
                                          max_seq_len=max_seq_len, validate=validate)
        starts = [0]
        for v in q_lengths:
            starts.append(starts[-1] + v)
        loc = torch.tensor(starts, dtype=torch.int32).to(query.device)
        if max_query_len is None:
            max_query_len = max(q_lengths, default=0)
    else:
        if query_start_loc.ndim != 1 or query_start_loc.numel() < 1:
            raise ValueError("query_start_loc must have shape [batch + 1]")
        batch = query_start_loc.numel() - 1
        loc = query_start_loc.to(device=query.device, dtype=torch.int32).contiguous()
        if max_query_len is None:
            max_query_len = int((loc[1:] - loc[:-1]).max().item()) if batch else 0
    if block_table.ndim != 2 or block_table.shape[0] < batch:
        raise ValueError("block_table must have shape [batch, max_blocks]")
    block_size = key_cache.shape[1]
    if isinstance(seq_lens, torch.Tensor):
        lens_dev = seq_lens.to(device=query.device, dtype=torch.int32).contiguous()
        if lens_dev.numel() < batch:
            raise ValueError("one sequence length is required per request")
        if max_seq_len is None:
            max_seq_len = int(lens_dev[:batch].max().item()) if batch else 0
    else:
        lengths = [int(v) for v in seq_lens]
        if len(lengths) != batch:
            raise ValueError("one sequence length is required per request")
        if any(v < 0 for v in lengths):
            raise ValueError("sequence lengths must be non-negative")
        lens_dev = torch.tensor(lengths, dtype=torch.int32).to(query.device)
        if max_seq_len is None:
            max_seq_len = max(lengths, default=0)
    if max_seq_len > block_table.shape[1] * block_size:
        raise ValueError("block_table has too few entries for a sequence length")
    table = block_table[:batch]
    if table.dtype not in (torch.int32, torch.int64):
        table = table.to(torch.int64)
    table = table.to(query.device).contiguous()
    if validate and batch:
        # A max_query_len below the longest request would leave that request's
        # later rows unwritten (the grid is sized by it).
        longest = int((loc[1:batch + 1] - loc[:batch]).max().item())
        if longest > max_query_len:
            raise ValueError(f"max_query_len ({max_query_len}) is smaller than a request's query length ({longest})")
    if validate and batch and max_seq_len > 0:
        if bool((lens_dev[:batch] > max_seq_len).any()):
            raise ValueError("max_seq_len is smaller than a sequence length")
        needed = (max_seq_len + block_size - 1) // block_size
        used = (torch.arange(needed, device=query.device)[None, :] * block_size
                < lens_dev[:batch, None].to(torch.int64))
        ids = table[:, :needed].to(torch.int64)
        if bool(((ids < 0) | (ids >= key_cache.shape[0]))[used].any()):
            raise IndexError("block_table references a block outside the cache")
    extension = native.load_extension()
    return native._operator("hif8_paged_prefill_attention", extension)(
        query.contiguous(), key_cache, value_cache, table, loc, lens_dev, float(scale), int(max_query_len),
        int(max_seq_len), bool(causal))


__all__ = [
    "HIF8_CACHE_DTYPE",
    "HIF8_SCALE_BYTES",
    "Hif8KVCacheLayout",
    "pack_kv_rows",
    "paged_attention",
    "paged_decode_attention",
    "unpack_kv_rows",
    "write_kv_cache",
]
