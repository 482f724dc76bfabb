"""Torch-CPU restatement of the reference's CPU GEMV path, for the timed CPU
baseline.

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module: it is the baseline that is timed on the
GPU box's host cores, never part of the product.

It restates, with torch CPU tensor ops so that it runs on every host thread
that ``torch.set_num_threads`` grants:

* the static activation quant of the reference's CPU oracle
  (``calibration.saturating_encode_tensor`` / ``static_quantize_tensor``,
  calibration.py:139-201, with the vectorised encode of
  ``torch_codec.encode_tensor``, torch_codec.py:32-49): divide by the scale in
  FP32, clamp finite values to +-2^15, index the 4096-entry magnitude table by
  (exponent, top four mantissa bits), sign except for zero, Inf / NaN by the
  full mantissa;
* the soft-decode GEMV of the reference's op test
  (tests/test_npu_ops.py:334-336): decode-table activations times their row
  scale, decode-table weights times their channel scale, one FP32 matmul.

* the paged decode attention of the reference's CPU oracle
  (``paged_attention_reference``, kv_cache.py:314-372): gather each
  request's packed rows through the block table, split codes and the
  little-endian FP32 row scale, decode times scale, round to the query dtype,
  repeat the KV heads over their query-head group, softmax of the scaled
  logits in FP32 rounded back to the query dtype, then the weighted sum, with
  the query-dtype tensors torch itself computes on (one query row per
  request).

Pinned by ``tests/test_oracle_torch_cpu.py``: codes equal the numpy oracle's
``static_quant_rows`` bit for bit on every bf16 pattern and on random FP32
values, the GEMV is within FP32 rounding of ``linear_u8_u8`` (float64), and
the attention is within bf16 rounding of the numpy oracle's
``paged_attention_reference`` (float64 and bf16-rounding variants).
"""

from __future__ import annotations

import torch

from oracle import hif8_oracle as o

_MAG = torch.from_numpy(o.LUT4096.astype("int32"))
_DECODE = torch.from_numpy(o.DECODE_F32.copy())


def static_quant(x: torch.Tensor, scale) -> torch.Tensor:
    """Saturating static encode of ``x / scale`` (float32 division) -> uint8 codes.

    ``scale`` is one float or a float32 tensor broadcast against ``x`` (e.g.
    ``[rows, 1]`` for per-row weight scales)."""
    s = scale.to(torch.float32) if isinstance(scale, torch.Tensor) else torch.tensor(scale, dtype=torch.float32)
    q = x.to(torch.float32) / s
    finite = torch.isfinite(q)
    q = torch.where(finite, q.clamp(-o.MAX_FINITE, o.MAX_FINITE), q)
    bits = q.view(torch.int32)
    exponent = (bits >> 23) & 0xFF
    mantissa = bits & 0x7FFFFF
    sign = (bits >> 24) & 0x80
    mag = _MAG[exponent * 16 + (mantissa >> 19)]
    code = torch.where(mag == 0, mag, mag | sign)
    special = exponent == 0xFF
    code = torch.where(special, torch.where(mantissa != 0, torch.full_like(code, o.NAN_CODE), sign | o.PINF), code)
    return code.to(torch.uint8)


def soft_gemv(a_codes: torch.Tensor, a_scale: torch.Tensor, w_codes: torch.Tensor,
              w_scale: torch.Tensor) -> torch.Tensor:
    """(dec(a) * a_scale[:, None]) @ (dec(w) * w_scale[:, None])^T in FP32."""
    a = _DECODE[a_codes.to(torch.int32)] * a_scale.reshape(-1, 1)
    w = _DECODE[w_codes.to(torch.int32)] * w_scale.reshape(-1, 1)
    return a @ w.T


def paged_decode_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                           block_table: torch.Tensor, seq_lens, scale: float) -> torch.Tensor:
    """query [B, Hq, D] (bf16/fp16), caches [blocks, block_size, Hkv, D + 4] uint8,
    block_table [B, max_blocks]; one query row per request -> [B, Hq, Dv]."""
    block_size, hkv = key_cache.shape[1], key_cache.shape[2]
    d, dv = key_cache.shape[-1] - 4, value_cache.shape[-1] - 4
    flat_k = key_cache.reshape(-1, hkv, d + 4)
    flat_v = value_cache.reshape(-1, hkv, dv + 4)
    out = []
    for b, length in enumerate(int(v) for v in seq_lens):
        if length == 0:
            out.append(query.new_zeros(1, query.shape[1], dv))
            continue
        pos = torch.arange(length)
        slots = block_table[b, pos // block_size].to(torch.int64) * block_size + pos % block_size
        rows_k, rows_v = flat_k.index_select(0, slots), flat_v.index_select(0, slots)
        keys = (_DECODE[rows_k[..., :d].to(torch.int32)]
                * rows_k[..., d:].contiguous().view(torch.float32)).to(query.dtype)
        values = (_DECODE[rows_v[..., :dv].to(torch.int32)]
                  * rows_v[..., dv:].contiguous().view(torch.float32)).to(query.dtype)
        group = query.shape[1] // hkv
        keys = keys.repeat_interleave(group, dim=1)
        values = values.repeat_interleave(group, dim=1)
        logits = torch.einsum("qhd,khd->qhk", query[b:b + 1], keys) * float(scale)
        probs = torch.softmax(logits.float(), dim=-1).to(query.dtype)
        out.append(torch.einsum("qhk,khd->qhd", probs, values))
    return torch.cat(out, dim=0)
