"""CPU oracle for the HiF8 static W8A8KV8 hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker or the timed CPU baseline.  The product package never imports it and
has no CPU fallback.

This is a from-scratch numpy restatement of the reference's CPU algorithm.
Every function cites the reference file:line it follows (paths are relative to
the reference repository root).  Pinning (what independently checks each
function) is listed per function:

* value set / scalar codec          - golden table digests, exhaustive round trip,
                                      known-answer ties (tests/test_oracle_codec.py)
* LUTs (4096 / 8192 / static / bf16) - SHA-256 digests of the reference's generated
                                      table header (tests/golden/)
* vectorised encode                  - brute force against the scalar codec on every
                                      bf16 bit pattern and on random fp32 bits
* static quant                       - reference known answers + brute force
* linear_u8_u8                       - exact small-matrix known answer + fp64 brute force
* scaled decode                      - exhaustive 256 bytes x scale set, bf16 RNE
                                      checked against torch's own conversion
* KV pack/unpack/scatter/gather      - reference known answers (byte layout)
* paged attention                    - textbook softmax attention in float64; a
                                      pure-Python per-row loop twin; closed forms that
                                      fix the right-aligned causal mask (uniform keys:
                                      output = mean of the visible values)
* embedding gather-decode            - the reference formula executed by torch on the
                                      CPU (bf16 table, bf16 scale, bf16 product) and
                                      closed-form products
* dynamic quant                      - the reference's known-answer rows (test_npu_ops.py:
                                      30-50), scale = finite amax exactly, and the
                                      reciprocal path equal to the float64 division encode
                                      except within 2 ulp of a rounding midpoint
* dynamic fused linear               - fp64 brute force (division encode, decode, dot)
                                      and equality with dynamic quant on exact rows
"""

from __future__ import annotations

import bisect
import math
from typing import Sequence

import numpy as np

ZERO = 0x00
NAN_CODE = 0x80
PINF = 0x6F
NINF = 0xEF
SAT_CODE = 0x6E

MIN_FINITE = 2.0 ** -22
MAX_FINITE = 2.0 ** 15
UNDERFLOW_TIE = 2.0 ** -23
OVERFLOW_TIE = 1.25 * MAX_FINITE
SCALE_BYTES = 4


# ---------------------------------------------------------------------------
# Value set and scalar codec  (codec.py:27-187)
# ---------------------------------------------------------------------------

# Byte base for the three-mantissa-bit exponents -3..3 (codec.py:29-39).
_SMALL_EXPONENT_BASE = {0: 0x08, 1: 0x10, -1: 0x18, 2: 0x20, 3: 0x28, -2: 0x30, -3: 0x38}


def mantissa_bits(exponent: int) -> int:
    """Tapered precision: 3 bits for |e|<=3, 2 for |e|<=7, 1 for |e|<=15 (codec.py:52-60)."""
    a = abs(exponent)
    if a <= 3:
        return 3
    if a <= 7:
        return 2
    if a <= 15:
        return 1
    raise ValueError(f"exponent {exponent} outside the HiF8 normal range")


def normal_code(exponent: int, mantissa: int) -> int:
    """Seven-bit magnitude code of (1 + m/2^mb) * 2^e (codec.py:27-49)."""
    if -3 <= exponent <= 3:
        return _SMALL_EXPONENT_BASE[exponent] + mantissa
    if 4 <= exponent <= 7:
        return 0x40 + (exponent - 4) * 4 + mantissa
    if -7 <= exponent <= -4:
        return 0x50 + (-exponent - 4) * 4 + mantissa
    if 8 <= exponent <= 15:
        return 0x60 + (exponent - 8) * 2 + mantissa
    if -15 <= exponent <= -8:
        return 0x70 + (-exponent - 8) * 2 + mantissa
    raise ValueError(f"exponent {exponent} outside the HiF8 normal range")


def positive_value_set() -> list[tuple[float, int]]:
    """The 127 non-negative finite (value, code) pairs, ascending (codec.py:63-82)."""
    pairs = [(0.0, ZERO)]
    pairs += [(2.0 ** e, e + 23) for e in range(-22, -15)]
    for e in range(-15, 16):
        mb = mantissa_bits(e)
        for m in range(1 << mb):
            v = (1.0 + m / (1 << mb)) * 2.0 ** e
            if v < OVERFLOW_TIE:
                pairs.append((v, normal_code(e, m)))
    pairs.sort()
    assert len(pairs) == 127 and len({c for _, c in pairs}) == 127
    return pairs


POSITIVE = positive_value_set()
POSITIVE_VALUES = [v for v, _ in POSITIVE]
POSITIVE_CODES = [c for _, c in POSITIVE]


def _decode_table() -> np.ndarray:
    """byte -> float64 value; 0x80 is NaN, 0x6F/0xEF are +-Inf (codec.py:90-103)."""
    mag = {c: v for v, c in POSITIVE}
    mag[PINF] = math.inf
    out = np.empty(256, dtype=np.float64)
    for b in range(256):
        if b == NAN_CODE:
            out[b] = math.nan
        else:
            m = mag[b & 0x7F]
            out[b] = -m if b & 0x80 else m
    return out


DECODE = _decode_table()
DECODE_F32 = DECODE.astype(np.float32)


def encode_scalar(value: float) -> int:
    """Nearest HiF8 byte, ties away from zero, no signed zero (codec.py:148-180)."""
    value = float(value)
    if math.isnan(value):
        return NAN_CODE
    if math.isinf(value):
        return NINF if value < 0 else PINF
    mag = abs(value)
    if mag < UNDERFLOW_TIE:
        return ZERO
    if mag >= OVERFLOW_TIE:
        return NINF if value < 0 else PINF
    hi = bisect.bisect_left(POSITIVE_VALUES, mag)
    if hi == len(POSITIVE_VALUES):
        code = POSITIVE_CODES[-1]
    elif hi == 0:
        code = POSITIVE_CODES[0]
    else:
        lo = hi - 1
        code = POSITIVE_CODES[hi if POSITIVE_VALUES[hi] - mag <= mag - POSITIVE_VALUES[lo] else lo]
    if code == ZERO:
        return ZERO
    return code | (0x80 if value < 0 else 0)


def decode_scalar(byte: int) -> float:
    """codec.py:183-187."""
    if not isinstance(byte, int) or not 0 <= byte <= 255:
        raise ValueError(f"HiF8 byte must be an integer in [0, 255], got {byte!r}")
    return float(DECODE[byte])


def bf16_bits_of_decode(byte: int) -> int:
    """BF16 payload of a decoded byte, canonical NaN 0x7FC0 (codec.py:106-145; tablegen.py:63-74)."""
    v = DECODE[byte]
    if math.isnan(v):
        return 0x7FC0
    return int(np.array([v], dtype=np.float32).view(np.uint32)[0] >> 16)


def half_bits_of_decode(byte: int) -> int:
    """FP16 payload of a decoded byte, canonical NaN 0x7E00 (tablegen.py:77-81)."""
    v = DECODE[byte]
    if math.isnan(v):
        return 0x7E00
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


# ---------------------------------------------------------------------------
# Lookup tables  (torch_codec.py:19-29; tablegen.py:24-99)
# ---------------------------------------------------------------------------

def encode_lut4096() -> np.ndarray:
    """Magnitude code for every (exp8, top-4-mantissa) index (torch_codec.py:19-29)."""
    out = np.empty(4096, dtype=np.uint8)
    for i in range(4096):
        bits = np.uint32(((i >> 4) << 23) | ((i & 15) << 19))
        f = float(np.array([bits], dtype=np.uint32).view(np.float32)[0])
        out[i] = encode_scalar(f) & 0x7F
    return out


LUT4096 = encode_lut4096()


def signed_encode_lut8192() -> np.ndarray:
    """13-bit (sign, exp8, mant4) index -> byte; exp 0xFF: top-4 mantissa selects NaN (tablegen.py:24-37)."""
    out = np.empty(8192, dtype=np.uint8)
    for i in range(8192):
        sign = 0x80 if i & 0x1000 else 0
        mi = i & 0x0FFF
        if (mi >> 4) == 0xFF:
            out[i] = NAN_CODE if (mi & 15) else (PINF | sign)
        else:
            m = int(LUT4096[mi])
            out[i] = m if m == 0 else (m | sign)
    return out


def static_signed_encode_lut8192() -> np.ndarray:
    """Same as the signed LUT with finite overflow saturated to 0x6E|sign (tablegen.py:40-49)."""
    out = signed_encode_lut8192().copy()
    for i in range(8192):
        if ((i & 0x0FFF) >> 4) != 0xFF and (out[i] & 0x7F) == PINF:
            out[i] = (out[i] & 0x80) | SAT_CODE
    return out


SIGNED_LUT = signed_encode_lut8192()
STATIC_LUT = static_signed_encode_lut8192()


def encode_decode_bf16_lut(static: bool) -> np.ndarray:
    """13-bit FP32 index -> bf16 payload of the decoded code (tablegen.py:84-99)."""
    src = STATIC_LUT if static else SIGNED_LUT
    table = np.array([bf16_bits_of_decode(b) for b in range(256)], dtype=np.uint16)
    return table[src.astype(np.int64)]


def pack_u16x2(values: np.ndarray) -> np.ndarray:
    """Two uint16 per uint32, low half first (tablegen.py:59-60)."""
    v = np.asarray(values, dtype=np.uint32)
    return v[0::2] | (v[1::2] << 16)


# ---------------------------------------------------------------------------
# Vectorised encode and static quantisation
# (torch_codec.py:32-49; calibration.py:139-217; hif8_static_quant.cpp:67-89)
# ---------------------------------------------------------------------------

def encode_array(x: np.ndarray) -> np.ndarray:
    """Elementwise FP32 encode; NaN decided by the FULL mantissa (torch_codec.py:32-49)."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = f.view(np.uint32)
    exponent = (bits >> 23) & 0xFF
    mantissa = bits & 0x7FFFFF
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    mag = LUT4096[(exponent * 16 + (mantissa >> 19)).astype(np.int64)]
    signed = np.where(mag == 0, mag, mag | sign)
    special = exponent == 0xFF
    inf = (sign | PINF).astype(np.uint8)
    out = np.where(special, np.where(mantissa != 0, np.uint8(NAN_CODE), inf), signed)
    return out.astype(np.uint8)


def saturating_encode_array(x: np.ndarray) -> np.ndarray:
    """Clamp finite values to +-2^15 first, keep Inf/NaN (calibration.py:139-158)."""
    v = np.asarray(x, dtype=np.float32)
    clipped = np.where(np.isfinite(v), np.clip(v, -MAX_FINITE, MAX_FINITE), v).astype(np.float32)
    return encode_array(clipped)


def static_quant_rows(x: np.ndarray, fixed_scale: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The ``hif8_static_quant`` contract on [rows, K] input.

    Row r uses ``fixed_scale[r % S]`` (hif8_static_quant.cpp:76-78); values are
    divided in FP32 with IEEE rounding (calibration.py:201), then saturating
    encoded.  Returns (u8 [rows, K], f32 row_scale [rows]).
    """
    x = np.asarray(x, dtype=np.float32)
    k = x.shape[-1]
    rows = x.size // k if k else 0
    x2 = x.reshape(rows, k)
    s = np.asarray(fixed_scale, dtype=np.float32).reshape(-1)
    if s.size == 0 or rows % s.size:
        raise ValueError(f"fixed_scale count {s.size} must divide {rows} activation rows")
    row_scale = s[np.arange(rows) % s.size].astype(np.float32)
    with np.errstate(all="ignore"):
        q = x2 / row_scale[:, None]
    return saturating_encode_array(q).reshape(x.shape), row_scale


def static_quantize_tensor(x: np.ndarray, scale: np.ndarray, group_axis: int | None = None):
    """Per-tensor or per-group fixed scale (calibration.py:161-201)."""
    x = np.asarray(x, dtype=np.float32)
    fixed = np.asarray(scale, dtype=np.float32).reshape(-1)
    if fixed.size == 0 or not np.all(np.isfinite(fixed) & (fixed > 0)):
        raise ValueError("all static HiFloat8 scales must be finite and greater than zero")
    if group_axis is None:
        if fixed.size != 1:
            raise ValueError(f"per-tensor static quantization requires one scale, got {fixed.size}")
        view = fixed.reshape((1,) * x.ndim)
    else:
        axis = group_axis % x.ndim
        if fixed.size != x.shape[axis]:
            raise ValueError(f"scale count {fixed.size} does not match dimension {axis}")
        shape = [1] * x.ndim
        shape[axis] = fixed.size
        view = fixed.reshape(shape)
    with np.errstate(all="ignore"):
        return saturating_encode_array(x / view), fixed.copy()


def quantize_rows(rows: Sequence[Sequence[float]], scales: Sequence[float] | None = None):
    """Per-row amax->1.0 scaled encode (codec.py:205-255). Returns (data u8, scale f64)."""
    mat = [[float(v) for v in r] for r in rows]
    if scales is None:
        sc = []
        for r in mat:
            finite = [abs(v) for v in r if math.isfinite(v)]
            sc.append(max(max(finite, default=0.0), 1.0e-12))
    else:
        sc = [float(s) for s in scales]
    data = np.array([[encode_scalar(v / s) for v in r] for r, s in zip(mat, sc)], dtype=np.uint8)
    return data, np.array(sc, dtype=np.float64)


# ---------------------------------------------------------------------------
# Linear  (reference.py:10-43; test_npu_ops.py:334-336)
# ---------------------------------------------------------------------------

def linear_u8_u8(a: np.ndarray, a_scale, w: np.ndarray, w_scale, bias=None) -> np.ndarray:
    """y = (sum_k dec(a) dec(w)) * a_scale[m] * w_scale[n] (+ bias), float64 (reference.py:10-43)."""
    a = np.asarray(a, dtype=np.uint8)
    w = np.asarray(w, dtype=np.uint8)
    if a.shape[-1] != w.shape[-1]:
        raise ValueError(f"incompatible K dimensions: activation={a.shape[-1]}, weight={w.shape[-1]}")
    with np.errstate(all="ignore"):
        acc = DECODE[a.astype(np.int64)] @ DECODE[w.astype(np.int64)].T
        y = acc * np.asarray(a_scale, dtype=np.float64).reshape(-1, 1) * np.asarray(w_scale, dtype=np.float64).reshape(1, -1)
        if bias is not None:
            y = y + np.asarray(bias, dtype=np.float64).reshape(1, -1)
    return y


def dynamic_quant_rows(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The ``hif8_dynamic_quant`` contract on [rows, K] input.

    scale[r] = max(max |x[r, :]| over finite values, 1e-12) in float32
    (hif8_dynamic_quant.cpp:64-78 and 112-135: ReduceMax, non-finite values
    ignored, kScaleEpsilon = 1e-12 from hif8_codec.h:20).  For K % 32 == 0
    the kernel multiplies by the float32 reciprocal (Muls(normalized, 1/scale),
    hif8_dynamic_quant.cpp:137) and encodes through the signed table or the
    scalar encoder (:138-171); other K take the scalar path with a true
    division (:64-79).  Returns (u8 [rows, K], f32 scale [rows]).
    """
    x = np.asarray(x, dtype=np.float32)
    k = x.shape[-1]
    rows = x.size // k if k else 0
    x2 = x.reshape(rows, k)
    finite = np.isfinite(x2)
    amax = np.where(finite, np.abs(x2), np.float32(0)).max(axis=1).astype(np.float32)
    scale = np.maximum(amax, np.float32(1.0e-12)).astype(np.float32)
    with np.errstate(all="ignore"):
        if k % 32 == 0:
            q = x2 * (np.float32(1.0) / scale)[:, None]
        else:
            q = x2 / scale[:, None]
    return encode_array(q.astype(np.float32)).reshape(x.shape), scale


def soft_fused_linear_reference(x: np.ndarray, w: np.ndarray, w_scale, bias=None) -> np.ndarray:
    """``soft_hif8_fused_gemm`` with the dynamic scale, float64 accumulation.

    s[m] = max(finite amax of row m, 1e-12) (soft_hif8_fused_gemm.cpp:536-566);
    the activation is encoded with a true float32 division and decoded
    (:506-516); out = dot(dec(a), dec(w)) * channel_scale * s (+ bias) (:730-745).
    """
    x = np.asarray(x, dtype=np.float32)
    finite = np.isfinite(x)
    amax = np.where(finite, np.abs(x), np.float32(0)).max(axis=1).astype(np.float32)
    s = np.maximum(amax, np.float32(1.0e-12)).astype(np.float32)
    with np.errstate(all="ignore"):
        codes = encode_array((x / s[:, None]).astype(np.float32))
    return linear_u8_u8(codes, s.astype(np.float64), w, w_scale, bias)


def linear_u8_u8_pure(a, a_scale, w, w_scale, bias=None):
    """Pure-Python loop version of reference.py:10-43 for tiny cases (pins the numpy one)."""
    m, k = len(a), len(a[0])
    n = len(w)
    out = []
    for i in range(m):
        row = []
        for j in range(n):
            acc = 0.0
            for t in range(k):
                acc += decode_scalar(int(a[i][t])) * decode_scalar(int(w[j][t]))
            v = acc * float(a_scale[i]) * float(w_scale[j])
            if bias is not None:
                v += float(bias[j])
            row.append(v)
        out.append(row)
    return out


# ---------------------------------------------------------------------------
# bf16 helpers and scaled decode  (hif8_scaled_decode.cpp:56-125)
# ---------------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even FP32 -> BF16 payload; NaN -> 0x7FC0."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    b = f.view(np.uint32).astype(np.uint64)
    rounded = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(f), np.uint16(0x7FC0), rounded).astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def scaled_decode(data: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """bf16_RNE(fp32(dec(b)) * scale[row]) as bf16 bit patterns (hif8_scaled_decode.cpp:94-107)."""
    d = np.asarray(data, dtype=np.uint8)
    s = np.asarray(scale, dtype=np.float32).reshape(-1, 1)
    with np.errstate(all="ignore"):
        prod = DECODE_F32[d.astype(np.int64)] * s
    return f32_to_bf16_bits(prod)


# ---------------------------------------------------------------------------
# KV cache layout and ops  (kv_cache.py:26-372)
# ---------------------------------------------------------------------------

def pack_kv_rows(data: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """[T,H,D] u8 + [T,H] f32 -> [T,H,D+4] u8, scale little-endian after the codes (kv_cache.py:151-170)."""
    data = np.asarray(data, dtype=np.uint8)
    scale = np.ascontiguousarray(np.asarray(scale, dtype="<f4"))
    if data.shape[-1] % SCALE_BYTES:
        raise ValueError("head dimension must be divisible by four for inline scales")
    out = np.empty((*data.shape[:-1], data.shape[-1] + SCALE_BYTES), dtype=np.uint8)
    out[..., :-SCALE_BYTES] = data
    out[..., -SCALE_BYTES:] = scale.view(np.uint8).reshape(*scale.shape, SCALE_BYTES)
    return out


def unpack_kv_rows(packed: np.ndarray, head_size: int) -> tuple[np.ndarray, np.ndarray]:
    """kv_cache.py:173-184."""
    packed = np.asarray(packed, dtype=np.uint8)
    if packed.shape[-1] != head_size + SCALE_BYTES:
        raise ValueError(f"packed last dimension must be {head_size + SCALE_BYTES}, got {packed.shape[-1]}")
    data = packed[..., :head_size]
    scale = np.ascontiguousarray(packed[..., head_size:]).view("<f4").reshape(packed.shape[:-1])
    return data, scale.astype(np.float32)


def quantize_kv_rows_static(x: np.ndarray, head_scale: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Static KV write: rows [T*H, D] through static quant with scale[r % H] (kv_runtime.py:1168-1199)."""
    x = np.asarray(x, dtype=np.float32)
    t, h, d = x.shape
    data, row_scale = static_quant_rows(x.reshape(t * h, d), head_scale)
    return data.reshape(t, h, d), row_scale.reshape(t, h)


def scatter_kv_rows(cache: np.ndarray, rows: np.ndarray, slot_mapping: np.ndarray, block_size: int) -> None:
    """In-place slot scatter; negative slots skipped; block OOB -> IndexError (kv_cache.py:187-218)."""
    slots = np.asarray(slot_mapping, dtype=np.int64).reshape(-1)
    valid = slots >= 0
    if valid.any():
        vs = slots[valid]
        if np.any(vs // block_size >= cache.shape[0]):
            raise IndexError("slot_mapping references a block outside the cache")
        cache[vs // block_size, vs % block_size] = rows[valid]


def gather_kv_rows(cache: np.ndarray, block_table: np.ndarray, seq_lens, block_size: int) -> list[np.ndarray]:
    """Per-request rows, token order (kv_cache.py:221-252)."""
    out = []
    for b, length in enumerate(int(v) for v in seq_lens):
        if length < 0:
            raise ValueError("sequence lengths must be non-negative")
        blocks = (length + block_size - 1) // block_size
        if blocks > block_table.shape[1]:
            raise ValueError("block_table has too few entries for a sequence length")
        if length == 0:
            out.append(np.empty((0, *cache.shape[2:]), dtype=cache.dtype))
            continue
        ids = np.asarray(block_table[b, :blocks], dtype=np.int64)
        if np.any(ids < 0) or np.any(ids >= cache.shape[0]):
            raise IndexError("block_table references a block outside the cache")
        out.append(cache[ids].reshape(-1, *cache.shape[2:])[:length])
    return out


def gather_kv_rows_concat(cache, block_table, seq_lens, block_size: int) -> np.ndarray:
    """Request-major concatenation, byte-identical to gather_kv_rows (kv_cache.py:255-311)."""
    parts = gather_kv_rows(cache, block_table, seq_lens, block_size)
    if not parts:
        return np.empty((0, *cache.shape[2:]), dtype=cache.dtype)
    return np.concatenate(parts, axis=0)


def decode_kv_rows(data: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """fp32 dec(b) * scale[t,h] (kv_cache.py:137-148)."""
    with np.errstate(all="ignore"):
        return DECODE_F32[np.asarray(data).astype(np.int64)] * np.asarray(scale, dtype=np.float32)[..., None]


def paged_attention_reference(query: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                              block_table: np.ndarray, seq_lens, block_size: int, scale: float,
                              rounding: str = "bf16", query_lens=None, causal: bool = True,
                              dtype: str = "bf16") -> np.ndarray:
    """Paged attention over HiF8 pages (kv_cache.py:314-372).

    ``query`` holds bf16 values as float32.  Without ``query_lens`` it is
    [B, Hq, D], one query token per request (decode).  With ``query_lens`` it
    is [T, Hq, D] in the TND layout: request b owns the next query_lens[b]
    rows, and those rows are the LAST query_lens[b] positions of its
    seq_lens[b] cached tokens (kv_cache.py:321-346), so with ``causal`` query
    row i of request b sees keys 0 .. seq_lens[b] - query_lens[b] + i (the
    right-aligned mask of kv_cache.py:365-369; sparse_mode=3 in
    kv_runtime.py:1526-1540).  Without ``causal`` every row sees every key.

    ``dtype`` is the query dtype ("bf16" or "f16"): K/V rows are gathered,
    decoded as dtype_RNE(dec(b) * s_row) (``decode_kv_rows(...).to(
    query.dtype)``) and query head h attends KV head h // (Hq / Hkv), the head
    ``repeat_interleave`` gives it (kv_cache.py:355-363).  ``rounding="bf16"``
    reproduces the reference's intermediate roundings to the query dtype
    (logits, probabilities and output are query-dtype tensors in
    kv_cache.py:364-371; the name is kept from when only bf16 queries were
    covered); ``rounding="f64"`` keeps every intermediate after the K/V
    decode in float64.  A query row that sees no key (an empty request,
    or a row whose position is negative because query_lens[b] > seq_lens[b],
    which the reference's attention plan rejects, kv_runtime.py:626-633)
    yields zeros.
    """
    if dtype not in ("bf16", "f16"):
        raise ValueError("dtype must be 'bf16' or 'f16'")
    rnd = round_bf16 if dtype == "bf16" else round_f16
    q = np.asarray(query, dtype=np.float64)
    rows_total, hq, d = q.shape
    lengths = [int(v) for v in seq_lens]
    bsz = len(lengths)
    if query_lens is None:
        q_lengths = [1] * bsz
    else:
        q_lengths = [int(v) for v in query_lens]
    if len(q_lengths) != bsz or sum(q_lengths) != rows_total or any(v < 0 for v in q_lengths):
        raise ValueError("query_lens must describe every query row")
    kw = key_cache.shape[-1] - SCALE_BYTES
    vw = value_cache.shape[-1] - SCALE_BYTES
    krows = gather_kv_rows(key_cache, block_table, lengths, block_size)
    vrows = gather_kv_rows(value_cache, block_table, lengths, block_size)
    out = np.zeros((rows_total, hq, vw), dtype=np.float64)
    hkv = key_cache.shape[2]
    if hq % hkv:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    group = hq // hkv
    q0 = 0
    for b in range(bsz):
        ql, kl = q_lengths[b], lengths[b]
        rows = slice(q0, q0 + ql)
        q0 += ql
        if ql == 0 or kl == 0:
            continue
        kd, ks = unpack_kv_rows(krows[b], kw)
        vd, vs = unpack_kv_rows(vrows[b], vw)
        keys = rnd(decode_kv_rows(kd, ks)).astype(np.float64)             # [L, Hkv, D]
        vals = rnd(decode_kv_rows(vd, vs)).astype(np.float64)
        qg = q[rows].reshape(ql, hkv, group, d)                           # head h = j * group + g
        logits = np.einsum("qjgd,kjd->qjgk", qg, keys, optimize=True)     # [ql, Hkv, G, L]
        visible = np.ones((ql, kl), dtype=bool)
        if causal:
            positions = np.arange(ql) + kl - ql                           # right-aligned query positions
            visible = np.arange(kl)[None, :] <= positions[:, None]
        mask = visible[:, None, None, :]
        seen = visible.any(axis=1)                                        # rows with at least one key
        if rounding == "bf16":
            logits = rnd(logits).astype(np.float64)
            logits = rnd(logits * np.float32(scale)).astype(np.float64)
            logits = np.where(mask, logits, -np.inf)
            mx = logits.max(axis=-1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            with np.errstate(invalid="ignore"):
                e = np.exp((logits - mx).astype(np.float32)).astype(np.float64)
                probs = rnd(e / e.sum(axis=-1, keepdims=True)).astype(np.float64)
            probs = np.where(mask, probs, 0.0)
            res = np.einsum("qjgk,kjd->qjgd", probs, vals, optimize=True).reshape(ql, hq, vw)
            res = rnd(res)
        else:
            logits = np.where(mask, logits * scale, -np.inf)
            mx = logits.max(axis=-1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            e = np.where(mask, np.exp(logits - mx), 0.0)
            with np.errstate(invalid="ignore"):
                probs = e / e.sum(axis=-1, keepdims=True)
            probs = np.where(mask, probs, 0.0)
            res = np.einsum("qjgk,kjd->qjgd", probs, vals, optimize=True).reshape(ql, hq, vw)
        out[rows] = np.where(seen[:, None, None], res, 0.0)
    return out


def embedding_reference(weight: np.ndarray, weight_scale: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """Token-embedding gather-decode, as float32 holding bf16 values (scheme.py:121-131).

    rows = weight[ids], decoded through the bf16 table (exact: HiF8 is a subset of
    bf16); the row scale is rounded to bf16 first; the product of two bf16 values
    is exact in float32 and is rounded once to bf16 (torch's bf16 multiply).
    """
    weight = np.asarray(weight, np.uint8)
    ids = np.asarray(ids).reshape(-1)
    if ids.size and (ids.min() < 0 or ids.max() >= weight.shape[0]):
        raise IndexError("embedding ids outside the vocabulary")
    rows = DECODE_F32[weight[ids].astype(np.int64)]
    scale = round_bf16(np.asarray(weight_scale, np.float32).reshape(-1)[ids])
    with np.errstate(all="ignore"):
        return round_bf16((rows * scale[:, None]).astype(np.float32))
