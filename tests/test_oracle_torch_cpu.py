"""Pins the torch-CPU baseline port (oracle/torch_cpu.py) against the numpy
oracle: static-quant codes bit for bit on every bf16 pattern (several scales,
NaN / Inf / saturation included) and random FP32 values, and the soft-decode
GEMV within FP32 rounding of the float64 linear_u8_u8."""

import numpy as np
import torch

from oracle import hif8_oracle as o
from oracle import torch_cpu


def test_static_quant_codes_equal_the_numpy_oracle_on_every_bf16_pattern():
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = bits.to(torch.float32)
    for scale in (1.0, 3.0, 1e-3, 0.0625, 7.5e4):
        got = torch_cpu.static_quant(x, scale).numpy()
        want, _ = o.static_quant_rows(x.numpy().reshape(1, -1), np.array([scale], np.float32))
        assert np.array_equal(got, want.reshape(-1)), scale


def test_static_quant_codes_on_random_fp32():
    rng = np.random.default_rng(7)
    raw = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = torch.from_numpy(raw.copy())
    got = torch_cpu.static_quant(x, 0.37).numpy()
    want, _ = o.static_quant_rows(raw.reshape(1, -1), np.array([0.37], np.float32))
    assert np.array_equal(got, want.reshape(-1))


def test_soft_gemv_matches_linear_u8_u8():
    rng = np.random.default_rng(11)
    a = rng.integers(0, 111, (2, 512), dtype=np.uint8)
    w = rng.integers(0, 111, (96, 512), dtype=np.uint8)
    sa = (rng.random(2, dtype=np.float32) + 0.5) * 1e-2
    sw = (rng.random(96, dtype=np.float32) + 0.5) * 1e-3
    got = torch_cpu.soft_gemv(torch.from_numpy(a), torch.from_numpy(sa), torch.from_numpy(w),
                              torch.from_numpy(sw)).numpy()
    want = o.linear_u8_u8(a, sa, w, sw)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_static_quant_with_per_row_scales():
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((64, 300)) * 0.02).astype(np.float32)
    ws = (np.abs(w).max(axis=1) / 32768.0).astype(np.float32)
    got = torch_cpu.static_quant(torch.from_numpy(w), torch.from_numpy(ws).reshape(-1, 1)).numpy()
    want, _ = o.static_quant_rows(w, ws)
    assert np.array_equal(got, want)


def test_paged_decode_attention_matches_the_numpy_oracle():
    """The torch-CPU attention port against paged_attention_reference: within
    bf16 resolution of the float64 variant and closer still to the variant
    that rounds like the reference's bf16 tensors; empty requests give zeros."""
    rng = np.random.default_rng(9)
    hkv, group, d, bs, nb = 2, 4, 32, 8, 12
    kc = np.zeros((nb, bs, hkv, d + 4), np.uint8)
    vc = np.zeros_like(kc)
    for c in (kc, vc):
        vals = rng.standard_normal((nb * bs, hkv, d)).astype(np.float32)
        data, sc = o.quantize_kv_rows_static(vals, (np.abs(vals).max(axis=(0, 2)) / 32768.0).astype(np.float32))
        o.scatter_kv_rows(c, o.pack_kv_rows(data, sc), np.arange(nb * bs), bs)
    table = np.array([[3, 7, 1, 0], [11, 2, 5, 9], [4, 6, 8, 10]])
    lens = [29, 7, 0]
    q = torch.randn(3, hkv * group, d, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    got = torch_cpu.paged_decode_attention(q, torch.from_numpy(kc), torch.from_numpy(vc), torch.from_numpy(table),
                                           lens, 0.2).float().numpy()
    f64 = o.paged_attention_reference(q.float().numpy(), kc, vc, table, lens, bs, 0.2, rounding="f64")
    b16 = o.paged_attention_reference(q.float().numpy(), kc, vc, table, lens, bs, 0.2, rounding="bf16")
    assert not got[2].any()
    np.testing.assert_allclose(got, f64, rtol=2e-2, atol=2e-2)
    np.testing.assert_allclose(got, b16, rtol=1e-2, atol=1e-2)
