"""Pinning of the dynamic (per-row scale) quant oracle and the dynamic fused
linear oracle: the reference's known-answer rows (test_npu_ops.py:30-50), the
scale definition, and the float64 division encode the reference's own tests
compare against (codec.quantize_rows, codec.py:205-255)."""

import bisect
import math

import numpy as np
import pytest
import torch

from oracle import hif8_oracle as o

MIDPOINTS = sorted({(a + b) / 2 for a, b in zip(o.POSITIVE_VALUES, o.POSITIVE_VALUES[1:])} | {o.UNDERFLOW_TIE})


def _codec_rows(rows):
    """quantize_rows semantics: scale = max(finite amax, 1e-12), encode(v / scale) in float64."""
    data, scales = [], []
    for row in rows:
        finite = [abs(v) for v in row if math.isfinite(v)]
        scale = max(max(finite, default=0.0), 1.0e-12)
        scales.append(scale)
        data.append([o.encode_scalar(v / scale) for v in row])
    return np.array(data, dtype=np.uint8), np.array(scales, dtype=np.float64)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_known_answer_rows(dtype):
    rows = [
        [0.0, 1.0, -2.0, 4.0],
        [0.25, -0.5, 1.0, -4.0],
        [float("nan"), float("inf"), -float("inf"), 0.0],
        [2.0**-12, -(2.0**-11), 2.0**-10, -(2.0**-9)],
    ]
    rounded = torch.tensor(rows, dtype=dtype).float().numpy()
    data, scale = o.dynamic_quant_rows(rounded)
    want_data, want_scale = _codec_rows(rounded.tolist())
    np.testing.assert_array_equal(data, want_data)
    np.testing.assert_array_equal(scale.astype(np.float64), want_scale.astype(np.float32).astype(np.float64))
    # Closed forms: amax maps to +-1 (code 0x08), NaN/Inf keep their codes, an all
    # non-finite row falls back to the 1e-12 floor.
    assert data[0, 3] == 0x08 and data[1, 3] == 0x88
    assert list(data[2]) == [0x80, 0x6F, 0xEF, 0x00] and scale[2] == np.float32(1.0e-12)


def test_scale_is_the_finite_amax():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 96)) * np.exp(rng.uniform(-8, 8, (64, 1)))).astype(np.float32)
    x[3, 7] = np.nan
    x[9, 1] = np.inf
    x[9, 2] = -np.inf
    x[12] = 0.0
    _, scale = o.dynamic_quant_rows(x)
    finite = np.where(np.isfinite(x), np.abs(x), 0).max(axis=1)
    np.testing.assert_array_equal(scale, np.maximum(finite, np.float32(1e-12)).astype(np.float32))
    assert scale[12] == np.float32(1e-12)


def _near_midpoint(q: float, ulps: int = 2) -> bool:
    mag = abs(q)
    i = bisect.bisect_left(MIDPOINTS, mag)
    tol = ulps * np.spacing(np.float32(mag))
    return any(abs(mag - MIDPOINTS[j]) <= tol for j in (i - 1, i) if 0 <= j < len(MIDPOINTS))


@pytest.mark.parametrize("k", [64, 4096])
def test_reciprocal_path_equals_division_away_from_midpoints(k):
    rng = np.random.default_rng(k)
    x = rng.standard_normal((48, k)).astype(np.float32)
    x[::5] *= 1e-30  # rows in the denormal-power-of-two range of HiF8 after scaling
    cols = rng.choice(k, size=max(1, k // 1000), replace=False)
    x[1::2, cols] *= 50.0
    data, scale = o.dynamic_quant_rows(x)
    exact = x.astype(np.float64) / scale.astype(np.float64)[:, None]
    want = o.encode_array(exact.astype(np.float32))  # float32 division, then encode
    diff = np.argwhere(data != want)
    assert len(diff) <= 1e-3 * x.size
    for r, c in diff:
        assert _near_midpoint(exact[r, c]), (r, c, exact[r, c])


def test_division_path_for_k_not_multiple_of_32():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((8, 100)).astype(np.float32)
    data, scale = o.dynamic_quant_rows(x)
    want, _ = _codec_rows(x.tolist())
    # float32 division vs float64 division: equal except within an ulp of a midpoint
    for r, c in np.argwhere(data != want):
        assert _near_midpoint(float(x[r, c]) / float(scale[r]), ulps=1)


def test_fused_linear_reference_brute_force():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 40)).astype(np.float32) * 3
    w = rng.integers(0, 111, (5, 40), dtype=np.uint8)
    ws = rng.random(5).astype(np.float32) + 0.5
    bias = rng.standard_normal(5)
    got = o.soft_fused_linear_reference(x, w, ws, bias)
    for m in range(2):
        s = max(max(abs(float(v)) for v in x[m]), 1e-12)
        for n in range(5):
            acc = 0.0
            for kk in range(40):
                code = o.encode_scalar(float(np.float32(x[m, kk]) / np.float32(s)))
                acc += o.decode_scalar(code) * o.decode_scalar(int(w[n, kk]))
            want = acc * s * float(ws[n]) + bias[n]
            assert got[m, n] == pytest.approx(want, rel=1e-12, abs=1e-12)


def test_fused_linear_equals_dynamic_quant_then_linear_on_division_path():
    rng = np.random.default_rng(13)
    x = rng.standard_normal((2, 72)).astype(np.float32)  # 72 % 32 != 0: both divide
    w = rng.integers(0, 111, (6, 72), dtype=np.uint8)
    ws = rng.random(6).astype(np.float32)
    codes, s = o.dynamic_quant_rows(x)
    np.testing.assert_array_equal(o.soft_fused_linear_reference(x, w, ws), o.linear_u8_u8(codes, s, w, ws))
