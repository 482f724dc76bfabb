"""Paged HiF8 KV cache on the GPU against the oracle.

* hif8_kv_cache_write: cache bytes equal static quant -> pack -> slot scatter
  exactly (test_hif8_kv_npu.py:380-551 shape: 128 + 9 tokens, real layer-3
  per-head scales, a page boundary), including padding slots, specials, both
  slot dtypes, fp16 input and the any-shape kernel.
* hif8_paged_decode_attention: within rtol = atol = 1e-2 of
  paged_attention_reference (kv_cache.py:314-372) on the BASELINE decode
  configs (Hq 16, Hkv 4, D 256, page 128, ctx {512, 4096, 16384} x batch {1, 4},
  shuffled page table), plus ragged lengths, other head sizes, GQA groups,
  block sizes, fp16 queries, int64 tables and the any-shape kernel.  A
  tighter bound relative to the output's magnitude catches indexing errors
  that the absolute tolerance would hide.
"""

import math

import numpy as np
import pytest
import torch

from _kv import KEY_SCALES_L3, VALUE_SCALES_L3
from _kv import build_cache as _build_cache
from _kv import randn as _randn
from oracle import hif8_oracle as o

pytestmark = pytest.mark.gpu

HIF8_MAX = 32768.0


def _oracle_caches(key, value, ks, vs, slots, nb, bs, fill=0xA5):
    hkv = key.shape[1]
    caches = []
    for x, s in ((key, ks), (value, vs)):
        data, row_scale = o.quantize_kv_rows_static(x.float().numpy(), np.asarray(s, np.float32))
        cache = np.full((nb, bs, hkv, x.shape[2] + 4), fill, np.uint8)
        o.scatter_kv_rows(cache, o.pack_kv_rows(data, row_scale), np.asarray(slots), bs)
        caches.append(cache)
    return caches


def _gpu_write(device, key, value, ks, vs, slots, nb, bs, fill=0xA5, **kw):
    from hif8_rocm import kv_cache

    hkv = key.shape[1]
    kc = torch.full((nb, bs, hkv, key.shape[2] + 4), fill, dtype=torch.uint8, device=device)
    vc = torch.full((nb, bs, hkv, value.shape[2] + 4), fill, dtype=torch.uint8, device=device)
    kv_cache.write_kv_cache(key.to(device), value.to(device), kc, vc, slots.to(device),
                            torch.tensor(ks, dtype=torch.float32, device=device),
                            torch.tensor(vs, dtype=torch.float32, device=device), **kw)
    torch.cuda.synchronize()
    return kc.cpu().numpy(), vc.cpu().numpy()


def _assert_bytes(got, want, what):
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{what}: {len(bad)} byte mismatches, first at {bad[:4].tolist()}"


# ------------------------------------------------------------------ write

def test_write_production_shape_with_real_layer3_scales(native_ops, device):
    tokens, hkv, d, bs, nb = 128 + 9, 4, 256, 128, 3
    key = _randn((tokens, hkv, d), 20260822, 3.0)
    value = _randn((tokens, hkv, d), 20260823, 1.5)
    slots = torch.arange(tokens, dtype=torch.int64)
    kc, vc = _gpu_write(device, key, value, KEY_SCALES_L3, VALUE_SCALES_L3, slots, nb, bs)
    wk, wv = _oracle_caches(key, value, KEY_SCALES_L3, VALUE_SCALES_L3, slots.numpy(), nb, bs)
    _assert_bytes(kc, wk, "key cache")
    _assert_bytes(vc, wv, "value cache")
    # The sidecar is the head's scale, little-endian, on every written row.
    from hif8_rocm.kv_cache import unpack_kv_rows

    _, scale = unpack_kv_rows(torch.from_numpy(kc.reshape(-1, hkv, d + 4)[:tokens]), d)
    assert torch.equal(scale, torch.tensor(KEY_SCALES_L3).repeat(tokens, 1))


@pytest.mark.parametrize("dtype,slot_dtype", [(torch.bfloat16, torch.int32), (torch.float16, torch.int64)])
def test_write_shuffled_slots_padding_and_specials(native_ops, device, dtype, slot_dtype):
    tokens, hkv, d, bs, nb = 50, 4, 256, 16, 5
    key = _randn((tokens, hkv, d), 7, 2.0, dtype)
    value = _randn((tokens, hkv, d), 8, 0.5, dtype)
    big = 1.0e20 if dtype == torch.bfloat16 else 6.0e4
    specials = torch.tensor([float("nan"), float("inf"), -float("inf"), big, -big, 0.0, -0.0, 1.0e-30],
                            dtype=torch.float32).to(dtype)
    key[3, 1, :8] = specials
    value[10, 3, 100:108] = specials
    g = torch.Generator().manual_seed(9)
    slots = torch.randperm(nb * bs, generator=g)[:tokens].to(slot_dtype)
    slots[[0, 17, 49]] = -1
    ks, vs = [0.01, 0.5, 3.0e-5, 7.0], [1.0, 2.0 ** -12, 0.3, 1234.5]
    kc, vc = _gpu_write(device, key, value, ks, vs, slots, nb, bs)
    wk, wv = _oracle_caches(key, value, ks, vs, slots.numpy(), nb, bs)
    _assert_bytes(kc, wk, "key cache")
    _assert_bytes(vc, wv, "value cache")


@pytest.mark.parametrize("d,dv,hkv,bs", [(24, 16, 2, 4), (16, 24, 1, 4), (128, 128, 2, 8), (20, 20, 3, 5)])
def test_write_other_head_sizes(native_ops, device, d, dv, hkv, bs):
    tokens, nb = 19, 6
    key = _randn((tokens, hkv, d), 11)
    value = _randn((tokens, hkv, dv), 12)
    slots = torch.randperm(nb * bs, generator=torch.Generator().manual_seed(13))[:tokens]
    ks, vs = [0.02 * (h + 1) for h in range(hkv)], [0.03 / (h + 1) for h in range(hkv)]
    kc, vc = _gpu_write(device, key, value, ks, vs, slots, nb, bs)
    wk, wv = _oracle_caches(key, value, ks, vs, slots.numpy(), nb, bs)
    _assert_bytes(kc, wk, "key cache")
    _assert_bytes(vc, wv, "value cache")


def test_write_rejects_or_skips_slots_past_the_cache(native_ops, device):
    from hif8_rocm import kv_cache

    tokens, hkv, d, bs, nb = 6, 2, 64, 4, 2
    key, value = _randn((tokens, hkv, d), 1), _randn((tokens, hkv, d), 2)
    slots = torch.tensor([0, 3, 8, -1, 7, 100], dtype=torch.int64)
    with pytest.raises(IndexError, match="invalid block"):
        _gpu_write(device, key, value, [1.0, 1.0], [1.0, 1.0], slots, nb, bs)
    # Without host validation the device skips those tokens and counts them.
    kc = torch.zeros((nb, bs, hkv, d + 4), dtype=torch.uint8, device=device)
    vc = torch.zeros_like(kc)
    counter = torch.zeros(1, dtype=torch.int32, device=device)
    ones = torch.ones(hkv, dtype=torch.float32, device=device)
    torch.ops.vllm_ascend_hif8.hif8_kv_cache_write(key.to(device), value.to(device), kc, vc, slots.to(device),
                                                    ones, ones, counter)
    torch.cuda.synchronize()
    assert int(counter.item()) == 2
    wk, wv = _oracle_caches(key, value, [1.0, 1.0], [1.0, 1.0], np.where(slots.numpy() >= nb * bs, -1, slots.numpy()),
                            nb, bs, fill=0)
    _assert_bytes(kc.cpu().numpy(), wk, "key cache")
    _assert_bytes(vc.cpu().numpy(), wv, "value cache")


# -------------------------------------------------------------- attention

def _check_attention(device, lens, hq, hkv, d, bs, *, dtype=torch.bfloat16, bt_dtype=torch.int32, seed=0,
                     q_mul=1.0, dv=None, mixed=False, bound=2e-2, scales=None, kv_mul=(1.0, 1.0)):
    from hif8_rocm import kv_cache

    kc, vc, table = _build_cache(device, lens, hkv, d, bs, seed, dv=dv, bt_dtype=bt_dtype, mixed=mixed,
                                 scales=scales, kv_mul=kv_mul)
    q = _randn((len(lens), hq, d), seed + 1, q_mul, dtype)
    scale = 1.0 / math.sqrt(d)
    out = kv_cache.paged_decode_attention(q.to(device), kc, vc, table.to(device), lens, scale=scale)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    kcn, vcn, tn = kc.cpu().numpy(), vc.cpu().numpy(), table.numpy()
    # K/V (and, in the second oracle, every intermediate) rounded to the query dtype.
    qdt = "f16" if dtype == torch.float16 else "bf16"
    ref = o.paged_attention_reference(q.float().numpy(), kcn, vcn, tn, lens, bs, scale, rounding="f64", dtype=qdt)
    ref16 = o.paged_attention_reference(q.float().numpy(), kcn, vcn, tn, lens, bs, scale, rounding="bf16",
                                        dtype=qdt)
    if dtype == torch.float16:
        bound = min(bound, 5e-3)  # fp16 keeps 11 bits: V, P and the output round 8x finer than bf16
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2)
    if q_mul <= 1.0:
        # The bf16 variant also rounds the logits to bf16 (the reference's CPU
        # einsum); with sharply peaked logits that rounding alone moves the
        # weights by several percent, so it is compared on ordinary logits only.
        np.testing.assert_allclose(got, ref16, rtol=1e-2, atol=1e-2)
    # Per (request, head): error well below the output's own magnitude.
    err = np.abs(got - ref).max(axis=-1)
    mag = np.abs(ref).max(axis=-1)
    worst = float((err / np.maximum(mag, 1e-3)).max())
    print(f"lens={lens[:4]}.. hq={hq} hkv={hkv} d={d} bs={bs}: max err {float(err.max()):.3e}, "
          f"max err/|out| {worst:.3e}", flush=True)
    assert worst < bound, worst
    for b, n in enumerate(lens):
        if n == 0:
            assert not got[b].any()


@pytest.mark.parametrize("batch", [1, 4])
@pytest.mark.parametrize("ctx", [512, 4096, 16384])
def test_attention_decode_configs(native_ops, device, batch, ctx):
    _check_attention(device, [ctx] * batch, 16, 4, 256, 128, seed=ctx + batch)


def test_attention_with_real_layer3_scales(native_ops, device):
    """The reference's real layer-3 K/V scales (test_hif8_kv_npu.py:427-436;
    the exporter's convention, near amax / 12 rather than amax / 32768) on
    K ~ 3 N(0, 1), V ~ 1.5 N(0, 1): codes in HiF8's 3-bit-mantissa core and
    the tapered ends, against the float64 and bf16-rounding oracles.  q is
    scaled by 0.35 so that the logits keep a standard deviation near 1, where
    the bf16 logit rounding of the second oracle stays below the tolerance."""
    for lens, seed in (([4096] * 4, 31), ([16384, 700, 1], 32)):
        _check_attention(device, lens, 16, 4, 256, 128, seed=seed, q_mul=0.35,
                         scales=(KEY_SCALES_L3, VALUE_SCALES_L3), kv_mul=(3.0, 1.5))


def test_attention_ragged_lengths_and_empty_requests(native_ops, device):
    _check_attention(device, [0, 1, 31, 32, 33, 127, 129, 1000], 16, 4, 256, 128, seed=3)


def test_attention_ragged_few_splits_and_repeated(native_ops, device):
    # One-tile splits (at most 16 per request): empty, one-split and
    # many-split requests side by side, and repeated calls give equal bytes.
    from hif8_rocm import kv_cache

    lens = [0, 100, 512, 33, 64, 1]
    for seed in (11, 12):
        _check_attention(device, lens, 16, 4, 256, 128, seed=seed)
    kc, vc, table = _build_cache(device, lens, 4, 256, 128, 13)
    q = _randn((len(lens), 16, 256), 14).to(device)
    first = kv_cache.paged_decode_attention(q, kc, vc, table.to(device), lens, scale=0.0625)
    for _ in range(3):
        again = kv_cache.paged_decode_attention(q, kc, vc, table.to(device), lens, scale=0.0625)
        torch.cuda.synchronize()
        assert torch.equal(again, first)


def test_attention_multi_tile_splits_with_tails(native_ops, device):
    _check_attention(device, [16379, 16384, 9000, 1], 16, 4, 256, 128, seed=4)


def test_attention_peaked_softmax(native_ops, device):
    # Static per-head scales: K/V are decoded rounded exactly like the
    # reference, so even sharply peaked weights stay close to the oracle.
    _check_attention(device, [4096, 777], 16, 4, 256, 128, seed=5, q_mul=8.0, bound=1e-2)


def test_attention_rows_with_mixed_scales(native_ops, device):
    # Tiles whose rows carry other scales than the range's first token take
    # the per-row-scale path.
    _check_attention(device, [3000, 129, 64], 16, 4, 256, 128, seed=8, mixed=True)


@pytest.mark.parametrize("hq,hkv,d,bs,lens,bt_dtype", [
    (8, 2, 128, 16, [5, 300, 47], torch.int64),     # block size 16: per-token page lookups
    (16, 1, 64, 32, [100, 64], torch.int32),        # group 16
    (8, 8, 128, 64, [70, 1], torch.int64),          # group 1, two workgroup rows of KV heads
    (16, 4, 256, 48, [200, 97], torch.int32),       # block size not a multiple of 32
])
def test_attention_other_shapes(native_ops, device, hq, hkv, d, bs, lens, bt_dtype):
    _check_attention(device, lens, hq, hkv, d, bs, bt_dtype=bt_dtype, seed=hq + d + bs)


def test_attention_fp16_query(native_ops, device):
    """fp16 queries: K, V and the softmax weights round to fp16 (the reference's
    query.dtype), against the fp16-rounding oracles with a bound 4x tighter
    than bf16's; a mixed-scale cache keeps P' * row scale in bf16 and is held to
    the same bound; the any-shape kernel rounds K/V to fp16 too."""
    _check_attention(device, [513, 2000], 16, 4, 256, 128, dtype=torch.float16, seed=6)
    _check_attention(device, [3000, 129, 64], 16, 4, 256, 128, dtype=torch.float16, seed=9, mixed=True)
    _check_attention(device, [40, 17], 4, 2, 64, 8, dtype=torch.float16, dv=32, seed=10)


def test_attention_fp16_decode_and_multi_token_kernels_agree(native_ops, device):
    """One query row per request through the decode kernel and through the
    multi-token kernel (the op paged_attention routes q_len = 1 batches away
    from): both round V and P to fp16 for fp16 queries, so they agree to fp16
    resolution, not just to the 1e-2 tolerance."""
    lens = [700, 4096, 33]
    kc, vc, table = _build_cache(device, lens, 4, 256, 128, 41)
    q = _randn((len(lens), 16, 256), 42, 1.0, torch.float16).to(device)
    loc = torch.arange(len(lens) + 1, dtype=torch.int32, device=device)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=device)
    dec = torch.ops.vllm_ascend_hif8.hif8_paged_decode_attention(q, kc, vc, table.to(device), lens_d, 0.0625,
                                                                  max(lens))
    pre = torch.ops.vllm_ascend_hif8.hif8_paged_prefill_attention(q, kc, vc, table.to(device), loc, lens_d, 0.0625,
                                                                   1, max(lens), True)
    torch.cuda.synchronize()
    a, b = dec.float().cpu(), pre.float().cpu()
    rel = float(((a - b).abs().amax(dim=-1) / b.abs().amax(dim=-1).clamp_min(1e-3)).max())
    print(f"fp16 decode vs multi-token kernel: max err/|out| {rel:.2e}", flush=True)
    assert rel < 2e-3, rel


@pytest.mark.parametrize("hq,hkv,d,dv,bs,lens", [
    (4, 2, 24, 24, 4, [9, 3, 0]),      # head size outside the MFMA set
    (4, 2, 64, 32, 8, [40, 17]),       # head_size_v != head_size
    (20, 1, 64, 64, 16, [33]),         # group 20 > 16
])
def test_attention_any_shape_kernel(native_ops, device, hq, hkv, d, dv, bs, lens):
    _check_attention(device, lens, hq, hkv, d, bs, dv=dv, seed=d + dv)


def test_attention_rejects_invalid_block_ids(native_ops, device):
    from hif8_rocm import kv_cache

    kc, vc, table = _build_cache(device, [100], 4, 256, 128, 1)
    table[0, 0] = kc.shape[0] + 5
    q = _randn((1, 16, 256), 2).to(device)
    with pytest.raises(IndexError, match="outside the cache"):
        kv_cache.paged_decode_attention(q, kc, vc, table.to(device), [100], scale=0.0625)
