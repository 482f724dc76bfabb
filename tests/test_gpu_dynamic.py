"""Dynamic (per-row scale) quant and the dynamic fused GEMV on the GPU, the
legacy W8A8HIF8_SOFT path (test_npu_ops.py:30-50 and 448-500 shape):
quant bytes and row scales bit-exact against the oracle, fused outputs within
rtol = atol = 1e-2 of the float64 oracle."""

import numpy as np
import pytest
import torch

from oracle import hif8_oracle as o

pytestmark = pytest.mark.gpu
KNOWN_ROWS = [
    [0.0, 1.0, -2.0, 4.0],
    [0.25, -0.5, 1.0, -4.0],
    [float("nan"), float("inf"), -float("inf"), 0.0],
    [2.0**-12, -(2.0**-11), 2.0**-10, -(2.0**-9)],
]


def _rows(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g, dtype=torch.float32)
    flat = x.reshape(-1, shape[-1])
    flat[1::3] *= 1e-3
    flat[2::5, : max(1, shape[-1] // 500)] *= 60.0
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dynamic_quant_known_rows(native_ops, device, dtype):
    from hif8_rocm import native

    x = torch.tensor(KNOWN_ROWS, dtype=dtype)
    data, scale = native.dynamic_quant(x.to(device))
    want, want_scale = o.dynamic_quant_rows(x.float().numpy())
    np.testing.assert_array_equal(data.cpu().numpy(), want)
    np.testing.assert_array_equal(scale.cpu().numpy(), want_scale)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 4096), (4, 12288), (513, 4096), (7, 100), (5, 48), (3, 2, 64), (2, 36)])
def test_dynamic_quant_matches_oracle(native_ops, device, dtype, shape):
    from hif8_rocm import native

    x = _rows(shape, seed=sum(shape), dtype=dtype)
    if x.numel() > 8:
        x.view(-1)[3] = float("nan")
        x.view(-1)[5] = float("-inf")
    data, scale = native.dynamic_quant(x.to(device))
    want, want_scale = o.dynamic_quant_rows(x.float().numpy())
    torch.cuda.synchronize()
    assert data.shape == x.shape and scale.shape == (x.numel() // shape[-1],)
    np.testing.assert_array_equal(data.cpu().numpy(), want)
    np.testing.assert_array_equal(scale.cpu().numpy(), want_scale)


def test_dynamic_quant_rejects_bad_input(native_ops, device):
    from hif8_rocm import native

    with pytest.raises(RuntimeError, match="float16 or torch.bfloat16"):
        native.dynamic_quant(torch.zeros(2, 16, device=device))


@pytest.mark.parametrize("m,n,k", [(1, 128, 4096), (2, 128, 4096), (1, 128, 12288), (2, 300, 1024), (2, 37, 100),
                                   (1, 12288, 4096), (1, 8200, 12288)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dynamic_fused_gemv_matches_oracle(native_ops, device, m, n, k, dtype):
    from hif8_rocm import native

    g = torch.Generator().manual_seed(m * 7 + n + k)
    x = (torch.randn(m, k, generator=g) * 3).to(dtype)
    w = torch.randint(0, 111, (n, k), generator=g, dtype=torch.uint8)
    ws = (torch.rand(n, generator=g) + 0.01) * 1e-4  # keeps fp16 outputs finite
    bias = torch.randn(n, generator=g).to(dtype)
    y = native.soft_fused_linear(x.to(device), w.to(device), ws.to(device), bias.to(device), output_dtype=dtype)
    want = o.soft_fused_linear_reference(x.float().numpy(), w.numpy(), ws.numpy(),
                                         bias.float().numpy().astype(np.float64))
    torch.cuda.synchronize()
    torch.testing.assert_close(y.cpu().float(), torch.from_numpy(want.astype(np.float32)), rtol=1e-2, atol=1e-2)
    # The reference's own check: fused against dynamic quant then GEMM (rtol = atol = 8e-2).
    data, ts = native.dynamic_quant(x.to(device))
    two = native.soft_linear(data, w.to(device), ts, ws.to(device), bias.to(device), output_dtype=dtype)
    torch.testing.assert_close(y.float(), two.float(), rtol=8e-2, atol=8e-2)


def test_dynamic_fused_rejects_more_than_two_rows(native_ops, device):
    from hif8_rocm import native

    x = torch.zeros(3, 64, dtype=torch.bfloat16, device=device)
    w = torch.zeros(4, 64, dtype=torch.uint8, device=device)
    with pytest.raises(ValueError, match="M <= 2"):
        native.soft_fused_linear(x, w, torch.ones(4, device=device), output_dtype=torch.bfloat16)


@pytest.mark.parametrize("rows", [1, 2, 64])
@pytest.mark.parametrize("fused", ["0", "1"])
def test_soft_linear_method(native_ops, device, monkeypatch, rows, fused):
    from hif8_rocm import scheme

    monkeypatch.setenv("HIF8_SOFT_FUSED_GENERATION", fused)
    g = torch.Generator().manual_seed(rows)
    layer = torch.nn.Module()
    w = torch.randint(0, 111, (96, 256), generator=g, dtype=torch.uint8)
    ws = torch.rand(96, 1, generator=g) + 0.1
    layer.weight = torch.nn.Parameter(w.to(device), requires_grad=False)
    layer.weight_scale = torch.nn.Parameter(ws.to(device), requires_grad=False)
    method = scheme.W8A8HiFloat8SoftLinearMethod()
    method.process_weights_after_loading(layer)
    x = torch.randn(rows, 256, generator=g).to(torch.bfloat16)
    y = method.apply(layer, x.to(device))
    if rows <= 2 and fused == "1":
        want = o.soft_fused_linear_reference(x.float().numpy(), w.numpy(), ws.reshape(-1).numpy())
    else:
        codes, s = o.dynamic_quant_rows(x.float().numpy())
        want = o.linear_u8_u8(codes, s, w.numpy(), ws.reshape(-1).numpy())
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (rows, 96)
    torch.testing.assert_close(y.cpu().float(), torch.from_numpy(want.astype(np.float32)), rtol=1e-2, atol=1e-2)
