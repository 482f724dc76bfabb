"""hif8_static_quant and hif8_scaled_decode on the GPU against the oracle:
bit-exact bytes, scales and bf16 payloads (test_npu_ops.py:52-135 shape)."""

import math

import numpy as np
import pytest
import torch

from _data import bf16_activation, input_scale_of
from oracle import hif8_oracle as o

pytestmark = pytest.mark.gpu

SCALES = (1.0, 0.75, 2.0 ** -10, 3.0e-5, 1234.5, 1.0e-12, 7.1e-3)


def _bits_tensor(dtype):
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype)


def _run_quant(native, x, scales, device):
    from hif8_rocm import native as api

    data, row_scale = api.static_quant(x.to(device), torch.tensor(scales, dtype=torch.float32, device=device))
    torch.cuda.synchronize()
    return data.cpu().numpy(), row_scale.cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,k", [(256, 256), (4, 256), (1024, 64)])
def test_static_quant_every_input_pattern(native_ops, device, dtype, rows, k):
    # (256, 256) takes the LDS-table kernel, (4, 256) the arithmetic encoder.
    x = _bits_tensor(dtype)[: rows * k].reshape(rows, k)
    xf = x.float().numpy()
    for s in SCALES:
        data, row_scale = _run_quant(native_ops, x, [s], device)
        want, want_scale = o.static_quant_rows(xf, np.array([s], np.float32))
        bad = np.flatnonzero(data.reshape(-1) != want.reshape(-1))
        assert bad.size == 0, f"scale={s}: {bad.size} mismatches, first x={xf.reshape(-1)[bad[:4]]}"
        assert np.array_equal(row_scale, want_scale)


@pytest.mark.parametrize("k", [5, 31, 37, 4133])
def test_static_quant_unaligned_rows(native_ops, device, k):
    x = _bits_tensor(torch.bfloat16)[: 3 * k].reshape(3, k)
    for s in (0.5, 3.0e-5):
        data, _ = _run_quant(native_ops, x, [s], device)
        want, _ = o.static_quant_rows(x.float().numpy(), np.array([s], np.float32))
        assert np.array_equal(data, want)


def test_static_quant_reference_rows_and_row_scale(native_ops, device):
    rows = torch.tensor(
        [[0.0, 1.0, -2.0, 4.0, 1.0e20], [0.25, -0.5, 1.0, -4.0, -1.0e20],
         [float("nan"), float("inf"), -float("inf"), 0.0, 2.0],
         [2.0 ** -12, -(2.0 ** -11), 2.0 ** -10, -(2.0 ** -9), 1.0]], dtype=torch.bfloat16).reshape(2, 2, 5)
    data, row_scale = _run_quant(native_ops, rows, [0.5, 2.0], device)
    want, _ = o.static_quantize_tensor(rows.float().numpy(), np.array([0.5, 2.0], np.float32), group_axis=1)
    assert np.array_equal(data, want)
    assert row_scale.tolist() == [0.5, 2.0, 0.5, 2.0]


def test_static_quant_kv_rows_with_real_per_head_scales(native_ops, device):
    # Realistic layer-3 K scales (test_hif8_kv_npu.py:427-436), rows = tokens*heads.
    scales = [0.9432383179664612, 0.7343872785568237, 0.9391698241233826, 1.1160656213760376]
    x = (torch.randn(137, 4, 256, generator=torch.Generator().manual_seed(20260822)) * 3.0).to(torch.bfloat16)
    data, row_scale = _run_quant(native_ops, x.reshape(-1, 256), scales, device)
    want, want_scale = o.static_quant_rows(x.float().numpy().reshape(-1, 256), np.array(scales, np.float32))
    assert np.array_equal(data, want)
    assert np.array_equal(row_scale, want_scale)


@pytest.mark.parametrize("m,k,heavy", [(1, 4096, False), (4, 12288, False), (4096, 4096, False), (512, 4096, True)])
def test_static_quant_config_shapes(native_ops, device, m, k, heavy):
    x = bf16_activation(m, k, seed=20261201 + m + k, heavy_tail=heavy)
    s = input_scale_of(x)
    data, row_scale = _run_quant(native_ops, x, s.tolist(), device)
    want, _ = o.static_quant_rows(x.float().numpy(), s.numpy())
    assert np.array_equal(data, want)
    assert np.all(row_scale == s.numpy()[0])


def test_static_quant_is_deterministic_and_repeatable(native_ops, device):
    from hif8_rocm import native as api

    x = bf16_activation(333, 4096, seed=5).to(device)
    s = input_scale_of(x.cpu()).to(device)
    outs = [api.static_quant(x, s)[0] for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0], t) for t in outs[1:])


# ----------------------------------------------------------- scaled decode

def test_every_decode_byte(native_ops, device):
    data = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(1, 256).to(device)
    out = native_ops.hif8_scaled_decode(data, torch.tensor([1.5], device=device))
    torch.cuda.synchronize()
    vals = out.cpu().float().reshape(-1).tolist()
    for byte, v in enumerate(vals):
        want = o.decode_scalar(byte) * 1.5
        assert (math.isnan(v) and math.isnan(want)) or v == want, hex(byte)


@pytest.mark.parametrize("k", [31, 37, 256, 4096, 4128, 4133])
def test_scaled_decode_rounding_and_tails(native_ops, device, k):
    from hif8_rocm import native as api

    g = torch.Generator().manual_seed(42)
    scales = torch.cat((torch.tensor([0.0, -0.0, 1.0, -1.0, 0.1, 1.00390625, 2.0 ** -20, 2.0 ** 20,
                                      float("inf"), float("nan")]), torch.rand(54, generator=g) * 0.02))
    codes = ((torch.arange(scales.numel() * k).reshape(-1, k) * 73) % 256).to(torch.uint8)
    got = api.scaled_decode(codes.to(device), scales.to(device)).cpu().view(torch.int16).numpy().astype(np.uint16)
    want = o.scaled_decode(codes.numpy(), scales.numpy())
    assert np.array_equal(got, want)


def test_scaled_decode_inline_kv_sidecar_view(native_ops, device):
    from hif8_rocm import native as api

    packed = torch.randint(0, 256, (3 * 2, 260), dtype=torch.uint8, generator=torch.Generator().manual_seed(3))
    scale = torch.tensor([0.5, 0.75, 1.0, 1.25, 1.5, 2.0], dtype=torch.float32)
    view = packed.to(device)[:, :256]
    assert not view.is_contiguous()
    got = api.scaled_decode(view, scale.to(device)).cpu().view(torch.int16).numpy().astype(np.uint16)
    assert np.array_equal(got, o.scaled_decode(packed[:, :256].numpy(), scale.numpy()))
