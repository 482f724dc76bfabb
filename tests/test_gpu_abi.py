"""The C-ABI entry points called directly (ctypes, raw device pointers, the
null stream) on the GPU, against the oracle: soft_hif8_gemm without a
workspace (A decoded per tile) and soft_hif8_gemm_with_workspace (A decoded
once into the workspace, K split into FP32 partials for shapes with few
output tiles).  Tolerance rtol = atol = 1e-2
(test_npu_ops.py:216-446); the split result is deterministic bit for bit."""

import ctypes

import numpy as np
import pytest
import torch

from _data import random_codes
from conftest import PKG_ROOT
from oracle import hif8_oracle as o

pytestmark = pytest.mark.gpu
LIB = PKG_ROOT / "hif8_rocm" / "libhif8_rocm.so"
BF16 = 1  # HIF8_DTYPE_BF16


@pytest.fixture(scope="module")
def lib(native_ops):
    lib = ctypes.CDLL(str(LIB))
    lib.hif8_last_error.restype = ctypes.c_char_p
    lib.soft_hif8_gemm_workspace_size.argtypes = [ctypes.c_int64] * 3
    lib.soft_hif8_gemm_workspace_size.restype = ctypes.c_size_t
    common = [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int] + [ctypes.c_int64] * 3
    lib.soft_hif8_gemm.argtypes = common + [ctypes.c_void_p]
    lib.soft_hif8_gemm_with_workspace.argtypes = common + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    return lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("m,n,k", [(512, 4096, 4096), (512, 2048, 4096), (300, 1000, 2048), (4096, 2048, 2048),
                                   (600, 4096, 12288), (2048, 4096, 1024), (2100, 4000, 1024)])
def test_workspace_gemm_matches_plain_and_oracle(lib, device, m, n, k):
    a = random_codes((m, k), seed=m + k)
    w = random_codes((n, k), seed=n + 3 * k)
    g = np.random.default_rng(m * n)
    ts = ((g.random(m, dtype=np.float32) + 1.0) * 1e-3).astype(np.float32)
    cs = ((g.random(n, dtype=np.float32) + 1.0) * 1e-3).astype(np.float32)
    bias = (g.random(n, dtype=np.float32) - 0.5).astype(np.float32)
    ta, tw, tts, tcs = (torch.from_numpy(v).to(device) for v in (a, w, ts, cs))
    tb = torch.from_numpy(bias).to(torch.bfloat16).to(device)
    need = lib.soft_hif8_gemm_workspace_size(m, n, k)
    print(f"split-K case m={m} n={n} k={k} workspace={need}", flush=True)
    assert need > m * k * 2, "these shapes take the split or the weight-decode path"
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    outs = []
    for workspace in (None, ws, ws):
        y = torch.empty(m, n, dtype=torch.bfloat16, device=device)
        args = [_ptr(ta), _ptr(tw), _ptr(tts), _ptr(tcs), _ptr(tb), BF16, _ptr(y), BF16, m, n, k]
        torch.cuda.synchronize()
        if workspace is None:
            st = lib.soft_hif8_gemm(*args, None)
        else:
            st = lib.soft_hif8_gemm_with_workspace(*args, _ptr(workspace), need, None)
        assert st == 0, lib.hif8_last_error()
        torch.cuda.synchronize()
        outs.append(y.cpu().float())
    assert torch.equal(outs[1], outs[2])
    rounded = torch.from_numpy(bias).to(torch.bfloat16).double().numpy()
    want = o.linear_u8_u8(a, ts, w, cs, rounded)
    for y in outs[:2]:
        torch.testing.assert_close(y, torch.from_numpy(want.astype(np.float32)), rtol=1e-2, atol=1e-2)
    # Same FP32 products, different summation order: at most one bf16 rounding step apart.
    torch.testing.assert_close(outs[1], outs[0], rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(4, 4096, 4096), (3, 16400, 4096), (4, 1000, 1040), (2, 640, 4096)])
def test_static_fused_gemm_abi_equals_quant_then_gemm(lib, device, m, n, k, xdtype):
    """soft_hif8_static_fused_gemm through the C ABI launches the fused GEMV
    itself at every M <= 4 (the MFMA-4 kernel's fused kind at M = 4 and at
    M = 3 over N >= 16384 with K <= 4096): bit-equal to hif8_static_quant +
    soft_hif8_gemm, special values and quotients on encode-index boundaries
    included."""
    for f in (lib.soft_hif8_static_fused_gemm,):
        f.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p,
                                                                                  ctypes.c_int] + [ctypes.c_int64] * 3 + [ctypes.c_void_p]
    lib.hif8_static_quant.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                      ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    g = torch.Generator().manual_seed(m * 131 + n + k)
    x = torch.randn(m, k, generator=g) * 2.0
    j = torch.arange(min(k, 256))
    x[0, : j.numel()] = (1.0 + (2 * (j % 16) + 1) / 32.0) * torch.pow(2.0, (j % 7 - 3).float()) * 0.5
    x[m - 1, 1] = float("nan")
    x[0, 2] = 7.0e4 if xdtype == torch.bfloat16 else 6.0e4
    x = x.to(xdtype).to(device)
    w = torch.from_numpy(random_codes((n, k), seed=n + k)).to(device)
    fixed = torch.tensor([0.5], device=device)
    cs = (torch.rand(n, generator=g) * 1e-2 + 1e-3).to(device)
    xd = 1 if xdtype == torch.bfloat16 else 0
    codes = torch.empty(m, k, dtype=torch.uint8, device=device)
    rs = torch.empty(m, dtype=torch.float32, device=device)
    want = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    got = torch.empty_like(want)
    print(f"fused ABI case m={m} n={n} k={k} x={xdtype}", flush=True)
    torch.cuda.synchronize()
    assert lib.hif8_static_quant(_ptr(x), xd, m, k, _ptr(fixed), 1, _ptr(codes), _ptr(rs), None) == 0, \
        lib.hif8_last_error()
    assert lib.soft_hif8_gemm(_ptr(codes), _ptr(w), _ptr(rs), _ptr(cs), None, -1, _ptr(want), BF16, m, n, k,
                              None) == 0, lib.hif8_last_error()
    assert lib.soft_hif8_static_fused_gemm(_ptr(x), xd, _ptr(w), _ptr(fixed), _ptr(cs), None, -1, _ptr(got), BF16,
                                           m, n, k, None) == 0, lib.hif8_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
