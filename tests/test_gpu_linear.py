"""soft_hif8_gemv / soft_hif8_gemm / soft_hif8_static_fused_gemm on the GPU
against the oracle's linear_u8_u8 (test_npu_ops.py:179-750 shape).  Tolerance
rtol = atol = 1e-2 on bf16/fp16 outputs with FP32 accumulation; the fused path
must equal quant -> GEMM bit for bit."""

import math

import numpy as np
import pytest
import torch

from _data import LAYER_SHAPES, bf16_activation, c1_operands, hif8_weight, input_scale_of, random_codes
from oracle import hif8_oracle as o

pytestmark = pytest.mark.gpu
TOL = dict(rtol=1e-2, atol=1e-2)


def _t(a, device, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return (t.to(dtype) if dtype is not None else t).to(device)


def _check(actual: torch.Tensor, expected: np.ndarray, **tol):
    torch.testing.assert_close(actual.cpu().float(), torch.from_numpy(np.asarray(expected, np.float32)),
                               **(tol or TOL), equal_nan=True)


def test_gemv_propagates_special_codes(native_ops, device):
    one = o.encode_scalar(1.0)
    codes = [0x80, 0x6F, 0xEF]
    act = torch.tensor([[c, one] for c in codes], dtype=torch.uint8, device=device)
    weight = torch.tensor([[one, 0] for _ in codes], dtype=torch.uint8, device=device)
    ts = torch.tensor([1.5, 0.5, 2.0], device=device)
    cs = torch.ones(3, device=device)
    for row, code in enumerate(codes):
        for out_dtype in (torch.float16, torch.bfloat16):
            y = native_ops.soft_hif8_gemv(act[row:row + 1].clone(), weight, ts[row:row + 1].clone(), cs, None, out_dtype)
            torch.cuda.synchronize()
            got = y.cpu().float()[0, row].item()
            want = o.decode_scalar(code) * ts[row].item()
            assert (math.isnan(got) and math.isnan(want)) or got == want


@pytest.mark.parametrize("rows", [2, 3, 4])
def test_multi_row_gemv_propagates_special_codes(native_ops, device, rows):
    """M = 2..4 (the MFMA GEMV): NaN and +-Inf codes in the activation or the
    weight reach exactly the outputs they feed, in either output dtype."""
    one = o.encode_scalar(1.0)
    k, n = 64, 8
    act = np.zeros((rows, k), np.uint8)
    act[:, 5] = one
    weight = np.zeros((n, k), np.uint8)
    weight[:, 5] = one
    weight[1, 9] = 0x6F          # +Inf weight: meets activation zeros -> NaN in row 1 of every m
    act[rows - 1, 9] = one       # ... and 1.0 in the last activation row -> +Inf there
    weight[2, 5] = 0xEF          # -Inf weight times activation 1.0 -> -Inf
    act[0, 20] = 0x80            # NaN activation code: all of row m = 0 is NaN (NaN x 0 is NaN)
    weight[3, 20] = one
    ts = np.full(rows, 0.5, np.float32)
    cs = np.full(n, 2.0, np.float32)
    with np.errstate(all="ignore"):
        want = o.linear_u8_u8(act, ts, weight, cs)
    for out_dtype in (torch.float16, torch.bfloat16):
        y = native_ops.soft_hif8_gemm(_t(act, device), _t(weight, device), _t(ts, device), _t(cs, device), None,
                                      out_dtype)
        torch.cuda.synchronize()
        got = y.cpu().float().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(want)), (got, want)
        fin = ~np.isnan(want)
        assert np.array_equal(got[fin], want[fin].astype(np.float32)), (got, want)


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5])
def test_soft_linear_matches_reference_small(native_ops, device, rows):
    from hif8_rocm import native as api

    w, ws = o.quantize_rows([[1.0, -2.0, 0.5, 4.0], [-0.25, 1.5, -3.0, 2.0], [2.0, 0.0, -1.0, 0.25]])
    a, sa = o.quantize_rows([[0.5 * (r + 1), -1.0, 2.0, -0.25 * (r + 1)] for r in range(rows)])
    for bias_dtype in (None, torch.float16, torch.bfloat16):
        bias_vals = None if bias_dtype is None else [0.5, -1.0, 2.0]
        bias = None if bias_dtype is None else torch.tensor(bias_vals, dtype=bias_dtype, device=device)
        want = o.linear_u8_u8(a, sa, w, ws, bias_vals)
        for out_dtype in (torch.float16, torch.bfloat16):
            y = api.soft_linear(_t(a, device), _t(w, device), _t(sa, device, torch.float32),
                                _t(ws, device, torch.float32), bias, output_dtype=out_dtype)
            _check(y, want)


@pytest.mark.parametrize("rows,channels,k", [
    (1, 17, 37), (2, 17, 37), (3, 3, 4), (5, 16, 16), (3, 17, 37), (3, 256, 16),
    (3, 2176, 16), (5, 16, 255), (1, 17, 1024), (2, 17, 1037), (1, 33, 2048),
    (63, 16, 37), (64, 16, 64), (65, 17, 128), (129, 1024, 4097), (130, 300, 4096),
    (2, 40, 4112), (3, 24, 8192), (4, 9, 4096), (2, 1, 16), (3, 40, 256), (1, 70, 512), (4, 33, 2048),
])
def test_gemm_shapes_and_tails(native_ops, device, rows, channels, k):
    a = random_codes((rows, k), seed=rows * 7 + k)
    w = random_codes((channels, k), seed=channels * 5 + k)
    g = np.random.default_rng(rows + channels + k)
    ts = (g.random(rows, dtype=np.float32) + 1.0) * 1e-3
    cs = (g.random(channels, dtype=np.float32) + 1.0) * 1e-3
    bias = (g.random(channels, dtype=np.float32) - 0.5)
    want = o.linear_u8_u8(a, ts, w, cs, bias.astype(np.float64))
    for out_dtype in (torch.bfloat16, torch.float16):
        y = native_ops.soft_hif8_gemm(_t(a, device), _t(w, device), _t(ts, device), _t(cs, device),
                                      _t(bias, device, out_dtype), out_dtype)
        y2 = native_ops.soft_hif8_gemm(_t(a, device), _t(w, device), _t(ts, device), _t(cs, device),
                                       _t(bias, device, out_dtype), out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)
        rounded = bias.astype(np.float32)
        rounded = (torch.from_numpy(rounded).to(out_dtype).float().numpy()).astype(np.float64)
        _check(y, want - bias + rounded)


@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("n,k", LAYER_SHAPES)
def test_decode_gemv_config_shapes(native_ops, device, m, n, k):
    """M in {1,4} over one layer's projection shapes."""
    from hif8_rocm import native as api

    x = bf16_activation(m, k, seed=20261201 + k)
    s = input_scale_of(x)
    w, ws = hif8_weight(n, k, seed=n + k)
    xq, _ = o.static_quant_rows(x.float().numpy(), s.numpy())
    want = o.linear_u8_u8(xq, np.repeat(s.numpy(), m), w, ws)
    data, rs = api.static_quant(x.to(device), s.to(device))
    y = api.soft_linear(data, _t(w, device), rs, _t(ws, device), None, output_dtype=torch.bfloat16)
    _check(y, want)
    fused = api.soft_static_fused_linear(x.to(device), _t(w, device), s.to(device), _t(ws, device),
                                         None, output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(fused, y)


def test_cpu_reference_gemv_config(native_ops, device):
    """M = 1, N = 12288, K = 4096 from seeded fp32 weights
    (reference oracle form: tests/test_npu_ops.py:334-344).  The activation
    codes from hif8_static_quant are bit-exact against the oracle; every one
    of the 12288 outputs of soft_linear is within 1e-2 of linear_u8_u8."""
    from hif8_rocm import native as api

    x, s, _, wq, ws = c1_operands()
    xq, xs = o.static_quant_rows(x.float().numpy(), s.numpy())
    data, rs = api.static_quant(x.to(device), s.to(device))
    torch.cuda.synchronize()
    assert np.array_equal(data.cpu().numpy(), xq)
    assert np.array_equal(rs.cpu().numpy(), xs)
    y = api.soft_linear(data, _t(wq, device), rs, _t(ws, device), None, output_dtype=torch.bfloat16)
    assert tuple(y.shape) == (1, 12288) and y.dtype == torch.bfloat16
    _check(y, o.linear_u8_u8(xq, xs, wq, ws))
    fused = api.soft_static_fused_linear(x.to(device), _t(wq, device), s.to(device), _t(ws, device), None,
                                         output_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(fused, y)


@pytest.mark.parametrize("m", [512, 4096])
@pytest.mark.parametrize("n,k", [(4096, 4096), (2048, 4096), (4096, 12288), (24576, 4096)])
@pytest.mark.parametrize("heavy", [False, True])
def test_prefill_gemm_config_shapes(native_ops, device, m, n, k, heavy):
    """BASELINE configs[2] shapes at full size: 48 sampled rows against the float64
    oracle, and every output against an FP32 product of the decoded operands."""
    from hif8_rocm import native as api

    x = bf16_activation(m, k, seed=m + n + k, heavy_tail=heavy)
    s = input_scale_of(x)
    w, ws = hif8_weight(n, k, seed=n * 3 + k)
    data, rs = api.static_quant(x.to(device), s.to(device))
    y = api.soft_linear(data, _t(w, device), rs, _t(ws, device), None, output_dtype=torch.bfloat16)
    rows = np.random.default_rng(m).choice(m, size=min(m, 48), replace=False)
    xq = data.cpu().numpy()[rows]
    want = o.linear_u8_u8(xq, np.repeat(s.numpy(), rows.size), w, ws)
    _check(y[torch.from_numpy(rows).to(device)], want)
    # Every output against an FP32 product of the decoded operands on the GPU
    # (the oracle's decode table; pinned to the float64 oracle by the rows
    # above), so a wrong tile or split anywhere in the M x N output fails.
    table = torch.from_numpy(o.DECODE_F32).to(device)
    allow = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        a32 = table[data.long()] * rs.reshape(-1, 1)
        w32 = table[_t(w, device).long()] * _t(ws, device).reshape(-1, 1)
        ref = a32 @ w32.T
    finally:
        torch.backends.cuda.matmul.allow_tf32 = allow
    torch.testing.assert_close(y.float(), ref, **TOL, equal_nan=True)


def test_static_fused_matches_static_quant_then_gemm(native_ops, device):
    g = torch.Generator().manual_seed(20260821)
    for rows, channels, k, with_bias in ((1, 128, 2048, False), (2, 256, 4096, True), (4, 256, 4096, True),
                                         (1, 128, 12288, True), (3, 77, 48, True), (1, 12288, 512, True),
                                         (1, 200, 5000, True), (1, 16400, 8192, False), (1, 300, 4100, True),
                                         (1, 64, 1000, False)):
        x = (torch.randn(rows, k, generator=g) * 3.0).to(torch.bfloat16).to(device)
        w = torch.randint(0, 111, (channels, k), generator=g, dtype=torch.uint8).to(device)
        fixed = torch.tensor([0.75], device=device)
        cs = (torch.rand(channels, generator=g) + 0.01).to(device)
        bias = torch.randn(channels, generator=g).to(torch.bfloat16).to(device) if with_bias else None
        data, row_scale = native_ops.hif8_static_quant(x, fixed)
        want = native_ops.soft_hif8_gemm(data, w, row_scale.contiguous(), cs, bias, torch.bfloat16)
        got = native_ops.soft_hif8_static_fused_gemm(x, w, fixed, cs, bias, torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (rows, channels, k)


@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,channels,k", [(4, 256, 4096), (4, 136, 1040), (3, 16400, 4096), (4, 40, 64),
                                             (2, 64, 4096), (3, 96, 2048)])
def test_static_fused_multi_row_equals_quant_then_gemm(native_ops, device, rows, channels, k, xdtype):
    """Several rows through the fused op - one launch of the MFMA-4 kernel's
    fused kind where it is the plan (K <= 4096 at M = 4, or M = 3 over
    N >= 16384), quant + GEMV otherwise - give the two-stage outputs bit for
    bit, NaN / Inf / saturating values, quotients at encode-index boundaries,
    all-zero-code rows, partial passes and row tails included."""
    g = torch.Generator().manual_seed(rows * 7919 + channels * 31 + k)
    x = torch.randn(rows, k, generator=g) * 3.0
    fixed = torch.tensor([0.75])
    # Quotients exactly on index boundaries: (1 + (2j + 1) / 32) * 2^e * s
    # are the midpoints between neighbouring three-bit mantissas.
    j = torch.arange(min(k, 512))
    x[0, : j.numel()] = (1.0 + (2 * (j % 16) + 1) / 32.0) * torch.pow(2.0, (j % 9 - 4).float()) * 0.75
    x[rows - 1, 3] = float("nan")
    x[rows - 1, 5] = float("inf")
    x[rows - 1, 7] = -float("inf")
    x[min(1, rows - 1), 9] = 1.0e5
    if rows >= 3:
        x[2] = torch.randn(k, generator=g) * 1.0e-9  # every code of this row is zero
    x = x.to(xdtype).to(device)
    w = torch.randint(0, 111, (channels, k), generator=g, dtype=torch.uint8)
    w[:, 5] = 0  # keep Inf x 0 away from every row but one column
    w[0, 5] = 8
    w = w.to(device)
    cs = (torch.rand(channels, generator=g) + 0.01).to(device)
    bias = torch.randn(channels, generator=g).to(torch.bfloat16).to(device)
    fixed = fixed.to(device)
    data, row_scale = native_ops.hif8_static_quant(x, fixed)
    for out_dtype in (torch.bfloat16, torch.float16):
        want = native_ops.soft_hif8_gemm(data, w, row_scale.contiguous(), cs, bias, out_dtype)
        got = native_ops.soft_hif8_static_fused_gemm(x, w, fixed, cs, bias, out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (rows, channels, k, out_dtype)


def test_static_fused_saturates_finite_outliers(native_ops, device):
    k = 2048
    x = torch.zeros((1, k), dtype=torch.bfloat16)
    x[0, :6] = torch.tensor([1.0e20, -1.0e20, 32768.0, -32768.0, 65536.0, -65536.0], dtype=torch.bfloat16)
    x = x.to(device)
    w = torch.zeros((128, k), dtype=torch.uint8, device=device)
    for c in range(6):
        w[c, c] = o.encode_scalar(1.0)
    fixed = torch.ones(1, device=device)
    cs = torch.ones(128, device=device)
    data, rs = native_ops.hif8_static_quant(x, fixed)
    want = native_ops.soft_hif8_gemm(data, w, rs, cs, None, torch.bfloat16)
    got = native_ops.soft_hif8_static_fused_gemm(x, w, fixed, cs, None, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert got[0, :6].float().tolist() == [32768.0, -32768.0, 32768.0, -32768.0, 32768.0, -32768.0]


def test_operator_row_contracts_are_strict(native_ops, device):
    act = torch.zeros((3, 4), dtype=torch.uint8, device=device)
    w = torch.zeros((2, 4), dtype=torch.uint8, device=device)
    with pytest.raises(RuntimeError, match="M <= 2"):
        native_ops.soft_hif8_gemv(act, w, torch.ones(3, device=device), torch.ones(2, device=device), None, torch.float16)


def test_nonzero_storage_offset_is_rejected(native_ops, device):
    view = torch.zeros((3, 4), dtype=torch.uint8, device=device)[1:]
    assert view.is_contiguous() and view.storage_offset() > 0
    with pytest.raises(RuntimeError, match="storage_offset == 0"):
        native_ops.soft_hif8_gemv(view, torch.zeros((2, 4), dtype=torch.uint8, device=device),
                                  torch.ones(2, device=device), torch.ones(2, device=device), None, torch.float16)


@pytest.mark.parametrize("n,k", LAYER_SHAPES)
def test_single_row_fusion_equals_the_two_stage_apply(native_ops, device, monkeypatch, n, k):
    """The scheme's default one-row route (the fused op) gives the two-stage
    route's outputs (HIF8_STATIC_FUSED_SINGLE_ROW=0) bit for bit at every
    decode projection shape."""
    import torch.nn as nn

    from hif8_rocm import scheme

    w, ws = hif8_weight(n, k, seed=n * 3 + k)
    x = bf16_activation(1, k, seed=k + 11)
    layer = nn.Module()
    layer.weight = nn.Parameter(_t(w, device), requires_grad=False)
    layer.weight_scale = nn.Parameter(_t(ws, device).reshape(-1, 1), requires_grad=False)
    layer.input_scale = nn.Parameter(input_scale_of(x).to(device), requires_grad=False)
    method = scheme.W8A8HiFloat8StaticLinearMethod()
    method.process_weights_after_loading(layer)
    monkeypatch.setenv("HIF8_STATIC_FUSED_SINGLE_ROW", "0")
    two_stage = method.apply(layer, x.to(device))
    monkeypatch.delenv("HIF8_STATIC_FUSED_SINGLE_ROW", raising=False)
    fused = method.apply(layer, x.to(device))
    torch.cuda.synchronize()
    assert torch.equal(fused, two_stage)


def test_decode_bf16_gives_every_code_exactly(native_ops, device):
    """hif8_decode_bf16 on all 256 codes (NaN 0x80 -> 0x7FC0) against the oracle's bf16 bits."""
    from hif8_rocm import native as api

    codes = np.tile(np.arange(256, dtype=np.uint8), 3).reshape(6, 128)
    got = api.decode_weight(_t(codes, device))
    torch.cuda.synchronize()
    bits = got.cpu().view(torch.int16).numpy().astype(np.uint16)
    want = np.array([o.bf16_bits_of_decode(int(c)) for c in codes.reshape(-1)], np.uint16).reshape(codes.shape)
    np.testing.assert_array_equal(bits, want)


@pytest.mark.parametrize("m,n,k", [(5, 16, 64), (129, 33, 128), (300, 1000, 2048), (512, 4096, 4096),
                                   (512, 4096, 12288), (2048, 24576, 256), (4096, 2048, 4096),
                                   (512, 24500, 256), (300, 24576, 128)])
def test_decoded_weight_gemm_matches_oracle_and_codes_path(native_ops, device, m, n, k):
    """soft_hif8_gemm_decoded_weight over hif8_decode_bf16(weight): within 1e-2 of the
    float64 oracle and within FP32 summation order of soft_hif8_gemm on the codes
    (split-K plans at M = 512, 128-, 256- and 256 x 192 tiles, ragged M and N)."""
    from hif8_rocm import native as api

    a = random_codes((m, k), seed=m + k)
    w, ws = hif8_weight(n, k, seed=n * 7 + k)
    g = np.random.default_rng(m * 3 + n)
    ts = (g.random(m, dtype=np.float32) + 0.5) * 1e-2
    bias = (g.random(n, dtype=np.float32) - 0.5)
    want = o.linear_u8_u8(a, ts, w, ws, bias.astype(np.float64))
    wd = api.decode_weight(_t(w, device))
    bias_t = _t(bias, device, torch.bfloat16)
    y = api.soft_linear_decoded_weight(_t(a, device), wd, _t(ts, device), _t(ws, device), bias_t,
                                       output_dtype=torch.bfloat16)
    y_codes = native_ops.soft_hif8_gemm(_t(a, device), _t(w, device), _t(ts, device), _t(ws, device), bias_t,
                                        torch.bfloat16)
    torch.cuda.synchronize()
    rounded = torch.from_numpy(bias).to(torch.bfloat16).float().numpy().astype(np.float64)
    _check(y, want - bias + rounded)
    torch.testing.assert_close(y.float(), y_codes.float(), rtol=1e-2, atol=1e-3)


def test_prefill_bf16_weights_scheme_equals_the_codes_scheme(native_ops, device, monkeypatch):
    """HIF8_PREFILL_BF16_WEIGHTS=1: the layer keeps a decoded weight; M > 4 runs on it
    (within FP32 summation order of the default), M <= 4 is unchanged bit for bit."""
    import torch.nn as nn

    from hif8_rocm import scheme

    n, k = 1000, 4096
    w, ws = hif8_weight(n, k, seed=5)

    def layer_with(flag):
        if flag:
            monkeypatch.setenv("HIF8_PREFILL_BF16_WEIGHTS", "1")
        else:
            monkeypatch.delenv("HIF8_PREFILL_BF16_WEIGHTS", raising=False)
        layer = nn.Module()
        layer.weight = nn.Parameter(_t(w, device), requires_grad=False)
        layer.weight_scale = nn.Parameter(_t(ws, device).reshape(-1, 1), requires_grad=False)
        layer.input_scale = nn.Parameter(torch.tensor([2e-4], device=device), requires_grad=False)
        method = scheme.W8A8HiFloat8StaticLinearMethod()
        method.process_weights_after_loading(layer)
        return method, layer

    m0, plain = layer_with(False)
    m1, cached = layer_with(True)
    assert plain._hif8_weight_bf16 is None and cached._hif8_weight_bf16.dtype == torch.bfloat16
    for rows in (3, 300):
        x = bf16_activation(rows, k, seed=rows).to(device)
        a, b = m0.apply(plain, x), m1.apply(cached, x)
        torch.cuda.synchronize()
        if rows <= 4:
            assert torch.equal(a, b)
        else:
            torch.testing.assert_close(b.float(), a.float(), rtol=1e-2, atol=1e-3)

