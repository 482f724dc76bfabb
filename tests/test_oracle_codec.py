"""Pins the CPU oracle's codec against the reference's golden tables, its
known-answer tests and brute force over the format's definition (CPU only)."""

import hashlib
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import hif8_oracle as o

GOLDEN = Path(__file__).resolve().parent / "golden" / "hif8_tables_digest.json"


def _digest(arr: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<")).tobytes()).hexdigest()


def _oracle_tables() -> dict:
    mag = o.DECODE_F32[:128].copy()
    bits = mag.view(np.uint32).copy()
    bits[np.isnan(mag)] = 0x7FC00000
    bf = np.array([o.bf16_bits_of_decode(b) for b in range(256)], np.uint16)
    hf = np.array([o.half_bits_of_decode(b) for b in range(256)], np.uint16)
    return {
        "kAscendDecodeMagnitude": bits,
        "kAscendDecodeBf16U16Packed": o.pack_u16x2(bf),
        "kAscendDecodeHalfU16Packed": o.pack_u16x2(hf),
        "kFloat32EncodeMagnitude": o.LUT4096,
        "kFloat32EncodeSignedU16Packed": o.pack_u16x2(o.SIGNED_LUT),
        "kFloat32StaticEncodeSignedU16Packed": o.pack_u16x2(o.STATIC_LUT),
        "kFloat32EncodeDecodeBf16U16Packed": o.pack_u16x2(o.encode_decode_bf16_lut(False)),
        "kFloat32StaticEncodeDecodeBf16U16Packed": o.pack_u16x2(o.encode_decode_bf16_lut(True)),
    }


@pytest.mark.parametrize("name", sorted(json.loads(GOLDEN.read_text())["tables"]))
def test_tables_match_reference_golden_digest(name):
    golden = json.loads(GOLDEN.read_text())["tables"][name]
    table = _oracle_tables()[name]
    assert table.size == golden["length"]
    assert _digest(table) == golden["sha256"]


# --- known answers restated from the reference's tests (test_codec.py:27-86) ---

def test_special_values():
    assert o.encode_scalar(0.0) == o.ZERO
    assert o.encode_scalar(-0.0) == o.ZERO
    assert o.encode_scalar(math.nan) == o.NAN_CODE
    assert o.encode_scalar(math.inf) == o.PINF
    assert o.encode_scalar(-math.inf) == o.NINF
    assert math.isnan(o.decode_scalar(o.NAN_CODE))
    assert o.decode_scalar(o.PINF) == math.inf
    assert o.decode_scalar(o.NINF) == -math.inf


def test_all_finite_codes_round_trip():
    assert len(o.POSITIVE) == 127
    for value, code in o.POSITIVE:
        assert o.encode_scalar(value) == code
        assert o.decode_scalar(code) == value
        if value:
            assert o.encode_scalar(-value) == code | 0x80
            assert o.decode_scalar(code | 0x80) == -value


def test_every_byte_has_defined_decode():
    for b in range(256):
        assert math.isnan(o.decode_scalar(b)) == (b == o.NAN_CODE)


def test_round_half_away_from_zero():
    assert o.decode_scalar(o.encode_scalar(1.0625)) == 1.125
    assert o.decode_scalar(o.encode_scalar(-1.0625)) == -1.125


def test_underflow_and_overflow_ties():
    assert o.encode_scalar(math.nextafter(o.UNDERFLOW_TIE, 0.0)) == o.ZERO
    assert o.decode_scalar(o.encode_scalar(o.UNDERFLOW_TIE)) == 2.0 ** -22
    assert o.decode_scalar(o.encode_scalar(math.nextafter(o.OVERFLOW_TIE, 0.0))) == o.MAX_FINITE
    assert o.encode_scalar(o.OVERFLOW_TIE) == o.PINF


def test_default_scaling_maps_amax_to_one():
    data, scale = o.quantize_rows([[0.0, -2.0, 1.0], [0.0, 0.0, 0.0]])
    assert scale[0] == 2.0
    assert o.decode_scalar(int(data[0][1])) == -1.0
    assert scale[1] > 0.0


def test_static_lut_only_saturates_finite_overflow():
    for i, (reg, sat) in enumerate(zip(o.SIGNED_LUT, o.STATIC_LUT)):
        if ((i & 0x0FFF) >> 4) == 0xFF:
            assert sat == reg
        elif (reg & 0x7F) == o.PINF:
            assert sat & 0x7F == 0x6E and sat & 0x80 == reg & 0x80
        else:
            assert sat == reg


# --- format definition checks independent of the oracle's encode implementation ---

def test_value_set_follows_tapered_precision():
    # Exponent range 2^-22 .. 2^15, precision 3/2/1 mantissa bits by |e|.
    vals = np.array(o.POSITIVE_VALUES[1:])
    assert vals.min() == 2.0 ** -22 and vals.max() == 2.0 ** 15
    for v in vals:
        e = math.floor(math.log2(v))
        frac = v / 2.0 ** e - 1.0
        bits = 0 if e < -15 else (3 if abs(e) <= 3 else 2 if abs(e) <= 7 else 1)
        assert (frac * (1 << bits)) == int(frac * (1 << bits))


def _nearest_by_definition(v: float) -> int:
    """argmin |v - value| with ties to the larger magnitude, straight from the spec."""
    if math.isnan(v):
        return o.NAN_CODE
    mag = abs(v)
    if mag >= o.OVERFLOW_TIE:
        return o.NINF if v < 0 else o.PINF
    values = np.array(o.POSITIVE_VALUES)
    d = np.abs(values - mag)
    best = np.flatnonzero(d == d.min()).max()
    code = o.POSITIVE_CODES[best]
    return 0 if code == 0 else code | (0x80 if v < 0 else 0)


def test_scalar_encode_is_nearest_ties_away_on_midpoints_and_random():
    rng = np.random.default_rng(20261201)
    vals = list(rng.standard_normal(300) * np.exp2(rng.integers(-25, 17, 300)))
    vals += [(a + b) / 2 for a, b in zip(o.POSITIVE_VALUES, o.POSITIVE_VALUES[1:])]
    for v in vals:
        for s in (1.0, -1.0):
            assert o.encode_scalar(s * v) == _nearest_by_definition(s * v), s * v


def test_vector_encode_matches_scalar_on_every_bf16_pattern():
    bits = (np.arange(65536, dtype=np.uint32) << 16)
    f = bits.view(np.float32)
    got = o.encode_array(f)
    want = np.array([o.encode_scalar(float(v)) for v in f], dtype=np.uint8)
    assert np.array_equal(got, want)


def test_vector_encode_matches_scalar_on_random_fp32_bits():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 120_000, dtype=np.uint64).astype(np.uint32)
    # Concentrate half of them in the HiF8 range (exponent fields 100..150).
    bits[::2] = (bits[::2] & 0x807FFFFF) | (rng.integers(100, 150, bits[::2].size, dtype=np.uint32) << 23)
    f = bits.view(np.float32)
    got = o.encode_array(f)
    want = np.array([o.encode_scalar(float(v)) for v in f], dtype=np.uint8)
    assert np.array_equal(got, want)


def test_nan_decided_by_full_mantissa():
    # A NaN whose top four mantissa bits are clear still encodes as NaN.
    f = np.array([0x7F800001, 0xFF810000, 0x7F800000, 0xFF800000], dtype=np.uint32).view(np.float32)
    assert list(o.encode_array(f)) == [0x80, 0x80, 0x6F, 0xEF]


def test_bf16_decode_is_exact_for_every_byte():
    for b in range(256):
        v = o.DECODE[b]
        bits = o.bf16_bits_of_decode(b)
        back = struct.unpack("<f", struct.pack("<I", bits << 16))[0]
        if math.isnan(v):
            assert bits == 0x7FC0
        else:
            assert back == v


# --- static quant (calibration.py:139-217; test_calibration.py:32-61) ---

def test_saturates_finite_outliers_but_preserves_special_values():
    src = np.array([-1e30, -o.MAX_FINITE, 0.0, o.MAX_FINITE, 1e30, -np.inf, np.inf, np.nan], np.float32)
    d = o.saturating_encode_array(src)
    assert d[0] == d[1] and d[3] == d[4]
    assert math.isfinite(o.decode_scalar(int(d[0]))) and math.isfinite(o.decode_scalar(int(d[4])))
    assert (d[5], d[6], d[7]) == (o.NINF, o.PINF, o.NAN_CODE)


def test_static_scalar_and_group_scales_round_trip():
    src = np.array([[[0.25, -0.5], [2.0, -4.0]], [[1.0, -2.0], [8.0, -16.0]]], np.float32)
    data, ret = o.static_quantize_tensor(src, np.array([2.0], np.float32))
    assert np.array_equal(ret, [2.0])
    assert np.array_equal(o.DECODE[data] * 2.0, src)  # all exactly representable
    grouped, _ = o.static_quantize_tensor(src, np.array([1.0, 4.0], np.float32), group_axis=1)
    assert np.array_equal(grouped[:, 0], o.static_quantize_tensor(src[:, 0], np.array([1.0], np.float32))[0])
    assert np.array_equal(grouped[:, 1], o.static_quantize_tensor(src[:, 1], np.array([4.0], np.float32))[0])


def test_rejects_invalid_scale_shapes_and_values():
    src = np.ones((2, 3), np.float32)
    with pytest.raises(ValueError):
        o.static_quantize_tensor(src, np.ones(2, np.float32))
    with pytest.raises(ValueError):
        o.static_quantize_tensor(src, np.ones(4, np.float32), group_axis=1)
    with pytest.raises(ValueError):
        o.static_quantize_tensor(src, np.array([0.0], np.float32))


def test_static_quant_rows_uses_row_modulo_scale():
    # test_npu_ops.py:52-75 shape: [2, 2, 5] rows with scales [0.5, 2.0].
    rows = np.array([[0.0, 1.0, -2.0, 4.0, 1e20], [0.25, -0.5, 1.0, -4.0, -1e20],
                     [np.nan, np.inf, -np.inf, 0.0, 2.0], [2.0 ** -12, -(2.0 ** -11), 2.0 ** -10, -(2.0 ** -9), 1.0]],
                    np.float32)
    fixed = np.array([0.5, 2.0], np.float32)
    data, row_scale = o.static_quant_rows(rows, fixed)
    assert np.array_equal(row_scale, [0.5, 2.0, 0.5, 2.0])
    grouped, _ = o.static_quantize_tensor(rows.reshape(2, 2, 5), fixed, group_axis=1)
    assert np.array_equal(data, grouped.reshape(4, 5))
    assert data[0, 4] == 0x6E and data[1, 4] == 0xEE  # saturated
    assert (data[2, 0], data[2, 1], data[2, 2]) == (0x80, 0x6F, 0xEF)


def test_static_quant_matches_scalar_codec_on_all_bf16_inputs():
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    for s in (1.0, 0.75, 2.0 ** -10, 3.0e-5, 1234.5):
        data, _ = o.static_quant_rows(x.reshape(1, -1), np.array([s], np.float32))
        with np.errstate(all="ignore"):
            q = x / np.float32(s)
        want = []
        for v in q:
            v = float(v)
            if math.isfinite(v):
                v = min(max(v, -o.MAX_FINITE), o.MAX_FINITE)
            want.append(o.encode_scalar(v))
        assert np.array_equal(data.reshape(-1), np.array(want, np.uint8)), s


def test_cpu_reference_config_weight_bytes_match_the_scalar_codec():
    """the fp32 weights' codes (row scale absmax / 32768)
    from the vectorised oracle equal the scalar codec on sampled rows, and
    each row's absmax lands exactly on the HiF8 maximum."""
    from _data import c1_operands

    x, s, w, wq, ws = c1_operands()
    assert w.shape == (12288, 4096) and wq.dtype == np.uint8 and ws.shape == (12288,)
    assert float(s[0]) == float(x.float().abs().max()) / 32768.0
    for r in np.random.default_rng(0).choice(12288, 6, replace=False):
        q = w[r] / ws[r]
        want = [o.encode_scalar(min(max(float(v), -o.MAX_FINITE), o.MAX_FINITE)) for v in q]
        assert np.array_equal(wq[r], np.array(want, np.uint8)), r
        assert o.SAT_CODE in (wq[r] & 0x7F)


# --- linear (reference.py:10-43; test_reference.py:8-12) ---

def test_exact_small_matrix():
    a, sa = o.quantize_rows([[1.0, 0.5], [-1.0, 0.25]])
    w, sw = o.quantize_rows([[1.0, 1.0], [0.5, -1.0]])
    out = o.linear_u8_u8(a, sa, w, sw, bias=[0.25, -0.5])
    assert out.tolist() == [[1.75, -0.5], [-0.5, -1.25]]
    assert o.linear_u8_u8_pure(a, sa, w, sw, [0.25, -0.5]) == [[1.75, -0.5], [-0.5, -1.25]]


def test_rejects_incompatible_shapes():
    a, sa = o.quantize_rows([[1.0, 2.0]])
    w, sw = o.quantize_rows([[1.0]])
    with pytest.raises(ValueError, match="incompatible K"):
        o.linear_u8_u8(a, sa, w, sw)


def test_numpy_linear_matches_pure_python_loops():
    rng = np.random.default_rng(3)
    a = rng.integers(0, 111, (3, 37), dtype=np.uint8)
    w = rng.integers(0, 111, (5, 37), dtype=np.uint8)
    sa, sw = rng.random(3) + 0.5, rng.random(5) + 0.5
    bias = rng.standard_normal(5)
    got = o.linear_u8_u8(a, sa, w, sw, bias)
    want = np.array(o.linear_u8_u8_pure(a, sa, w, sw, bias))
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_scaled_decode_rounds_like_torch():
    import torch

    codes = np.arange(256, dtype=np.uint8).reshape(1, 256).repeat(6, 0)
    scale = np.array([1.5, 0.1, 1.00390625, 2.0 ** -20, 0.0, np.inf], np.float32)
    got = o.scaled_decode(codes, scale)
    with np.errstate(all="ignore"):
        ref = torch.from_numpy(o.DECODE_F32[codes.astype(np.int64)] * scale[:, None]).to(torch.bfloat16)
    ref_bits = ref.view(torch.int16).numpy().astype(np.uint16)
    nan = np.isnan(ref.float().numpy())
    assert np.array_equal(got[~nan], ref_bits[~nan])
    assert np.all(got[nan] == 0x7FC0)


def test_embedding_reference_matches_torch_running_the_reference_formula():
    """scheme.py:121-131 executed literally by torch on the CPU: index_select,
    bf16 decode table, bf16(scale), bf16 product."""
    import torch

    rng = np.random.default_rng(11)
    vocab, dim = 300, 48
    weight = rng.integers(0, 256, (vocab, dim), dtype=np.uint8)
    scale = (rng.random(vocab, dtype=np.float32) * 3 + 1e-3).astype(np.float32)
    scale[:4] = [1.0, 0.5, 3.0e-7, 1234.5]
    ids = rng.integers(0, vocab, (5, 7))
    ids[0, :4] = [0, 1, 2, 3]
    want = o.embedding_reference(weight, scale, ids)
    lut = torch.tensor(o.DECODE, dtype=torch.bfloat16)
    flat = torch.from_numpy(ids.reshape(-1))
    rows = lut[torch.index_select(torch.from_numpy(weight), 0, flat).long()]
    ref = rows * torch.index_select(torch.from_numpy(scale), 0, flat).to(torch.bfloat16).unsqueeze(-1)
    got = torch.from_numpy(want)
    both_nan = torch.isnan(got) & torch.isnan(ref.float())
    assert torch.equal(got[~both_nan], ref.float()[~both_nan])
    # Closed forms: code of 1.5 times scale 2 is 3; NaN and Inf codes propagate.
    one5 = o.encode_scalar(1.5)
    w = np.array([[one5, o.NAN_CODE, 0x6F, 0x00]], np.uint8)
    out = o.embedding_reference(w, np.array([2.0], np.float32), np.array([0]))
    assert out[0, 0] == 3.0 and np.isnan(out[0, 1]) and out[0, 2] == np.inf and out[0, 3] == 0.0
    with pytest.raises(IndexError):
        o.embedding_reference(w, np.array([2.0], np.float32), np.array([1]))
