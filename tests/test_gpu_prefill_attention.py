"""Multi-token paged HiF8 attention (prefill / chunked prefill) on the GPU
against the oracle's paged_attention_reference with query_lens
(kv_cache.py:314-372; right-aligned causal mask kv_cache.py:365-369), within
rtol = atol = 1e-2 of the float64 oracle (and of the bf16-rounding oracle up
to that oracle's own distance from the float64 one).

Cases: BASELINE configs[3]'s cache shape (Hq 16, Hkv 4, D 256, 128-token
pages, shuffled page table) at q_len in {1, 17, 512} over ctx {512, 4096};
ragged batches with empty requests; causal off; rows whose positions precede
the first key; key splits with the combine; other head sizes, GQA groups and
block sizes; fp16 queries; int64 tables; mixed row scales; the any-shape
kernel.  Queries of more than two 64-row tiles (rows = tokens x query
heads per KV head) run the tile-image path, shorter ones the in-kernel page
decode; both appear above.  A bound relative to each output row's magnitude
catches indexing errors that the absolute tolerance would hide."""

import math

import numpy as np
import pytest
import torch

from _kv import KEY_SCALES_L3, VALUE_SCALES_L3, build_cache, randn
from oracle import hif8_oracle as o

pytestmark = pytest.mark.gpu


def _run_op(device, q, kc, vc, table, lens, qlens, scale, causal, max_query_len=None):
    """The torch op directly, with query_start_loc built from qlens (no routing)."""
    loc = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device=device)
    out = torch.ops.vllm_ascend_hif8.hif8_paged_prefill_attention(
        q.to(device), kc, vc, table.to(device), loc, torch.tensor(lens, dtype=torch.int32, device=device),
        scale, max(qlens) if max_query_len is None else max_query_len, max(lens), causal)
    torch.cuda.synchronize()
    return out


def _check(device, lens, qlens, hq, hkv, d, bs, *, causal=True, dtype=torch.bfloat16, bt_dtype=torch.int32,
           seed=0, dv=None, mixed=False, bound=2e-2, q_mul=1.0, via_api=False, scales=None, kv_mul=(1.0, 1.0)):
    from hif8_rocm import kv_cache

    kc, vc, table = build_cache(device, lens, hkv, d, bs, seed, dv=dv, bt_dtype=bt_dtype, mixed=mixed,
                                scales=scales, kv_mul=kv_mul)
    q = randn((sum(qlens), hq, d), seed + 1, q_mul, dtype)
    scale = 1.0 / math.sqrt(d)
    print(f"case lens={lens[:4]} qlens={qlens[:4]} hq={hq} hkv={hkv} d={d} bs={bs} causal={causal}", flush=True)
    if via_api:
        out = kv_cache.paged_attention(q.to(device), kc, vc, table.to(device), lens, scale=scale, query_lens=qlens,
                                       causal=causal)
        torch.cuda.synchronize()
    else:
        out = _run_op(device, q, kc, vc, table, lens, qlens, scale, causal)
    got = out.float().cpu().numpy()
    kcn, vcn, tn = kc.cpu().numpy(), vc.cpu().numpy(), table.numpy()
    qn = q.float().numpy()
    qdt = "f16" if dtype == torch.float16 else "bf16"   # K/V rounded to the query dtype
    if dtype == torch.float16:
        bound = min(bound, 5e-3)  # fp16 keeps 11 bits: V, P and the output round 8x finer than bf16
    ref = o.paged_attention_reference(qn, kcn, vcn, tn, lens, bs, scale, rounding="f64", query_lens=qlens,
                                      causal=causal, dtype=qdt)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2)
    if q_mul <= 1.0:
        # The bf16 variant rounds every logit to bf16 as the reference's CPU
        # einsum does; rows that see only a few keys turn that rounding into
        # weight changes of several percent, so each element may also differ
        # by the gap between the two oracles themselves.
        ref16 = o.paged_attention_reference(qn, kcn, vcn, tn, lens, bs, scale, rounding="bf16", query_lens=qlens,
                                            causal=causal, dtype=qdt)
        slack = np.abs(ref16 - ref)
        bad = np.abs(got - ref16) > 1e-2 + 1e-2 * np.abs(ref16) + slack
        assert not bad.any(), (int(bad.sum()), float(np.abs(got - ref16)[bad].max()))
    err = np.abs(got - ref).max(axis=-1)
    mag = np.abs(ref).max(axis=-1)
    worst = float((err / np.maximum(mag, 1e-3)).max())
    print(f"  max err {float(err.max()):.3e}, max err/|out| {worst:.3e}", flush=True)
    assert worst < bound, worst
    return got, ref


@pytest.mark.parametrize("ctx", [512, 4096])
@pytest.mark.parametrize("q_len", [1, 17, 512])
def test_prefill_config_shapes(native_ops, device, ctx, q_len):
    """q_len new tokens at the end of a ctx-token request (chunked prefill when
    q_len < ctx), next to a second request with its own shorter chunk."""
    second = max(1, q_len // 2)
    _check(device, [ctx, ctx // 2 + 3], [q_len, second], 16, 4, 256, 128, seed=ctx + q_len)


def test_prefill_from_empty_cache_whole_prompt(native_ops, device):
    # The usual prefill: every prompt token is a query row (q_len == seq_len).
    _check(device, [512, 300, 64], [512, 300, 64], 16, 4, 256, 128, seed=11)


def test_prefill_through_the_api_and_decode_routing(native_ops, device):
    _check(device, [700, 90], [33, 90], 16, 4, 256, 128, seed=12, via_api=True)
    # One row per request routes to the decode kernel and matches the oracle too.
    _check(device, [700, 90, 5], [1, 1, 1], 16, 4, 256, 128, seed=13, via_api=True)


def test_prefill_ragged_batch_with_empty_requests(native_ops, device):
    _check(device, [10, 0, 129, 300, 64, 1], [3, 0, 129, 65, 0, 1], 16, 4, 256, 128, seed=14)


def test_prefill_without_causal_mask(native_ops, device):
    _check(device, [300, 77], [40, 77], 16, 4, 256, 128, causal=False, seed=15)


def test_prefill_long_context_key_splits(native_ops, device):
    # Few query tiles over a long context: the key range is split over
    # workgroups and merged by the combine kernel.
    _check(device, [16384, 5000], [9, 64], 16, 4, 256, 128, seed=16)


def test_prefill_rows_before_the_first_key_are_zero(native_ops, device):
    # More query rows than cached tokens (the reference's plan rejects this;
    # the kernel gives the rows at negative positions zeros, like the oracle).
    got, _ = _check(device, [5, 40], [9, 40], 16, 4, 256, 128, seed=17)
    assert not got[:4].any()


@pytest.mark.parametrize("q_len", [17, 512])
def test_prefill_with_real_layer3_scales(native_ops, device, q_len):
    """The reference's real layer-3 K/V scales (test_hif8_kv_npu.py:427-436;
    near amax / 12, not amax / 32768) on K ~ 3 N(0, 1), V ~ 1.5 N(0, 1), over
    4096 cached keys: 17 rows run the in-kernel page decode, 512 the tile
    images."""
    _check(device, [4096, 1200], [q_len, min(q_len, 300)], 16, 4, 256, 128, seed=40 + q_len,
           scales=(KEY_SCALES_L3, VALUE_SCALES_L3), kv_mul=(3.0, 1.5))


def test_prefill_mixed_row_scales(native_ops, device):
    _check(device, [400, 129], [100, 20], 16, 4, 256, 128, seed=18, mixed=True)


def test_prefill_peaked_softmax(native_ops, device):
    _check(device, [1000, 300], [200, 31], 16, 4, 256, 128, seed=19, q_mul=8.0, bound=1e-2)


@pytest.mark.parametrize("qlen", [17, 200])
@pytest.mark.parametrize("order", ["rising", "falling"])
def test_prefill_scores_whose_max_keeps_growing(native_ops, device, qlen, order):
    """Scores that rise (or fall) along the keys by ~16 log2 units per 64-key
    tile: rising, every tile moves the softmax's running max by more than
    2^8, so the lazily updated reference and the rescale of O and l run at
    every tile; falling, the first tile holds the max and no rescale runs.
    Both the in-kernel path (17 tokens) and the tile-image path (200) take the
    same tile math; checked against the float64 oracle."""
    from hif8_rocm import kv_cache

    hq, hkv, d, bs = 16, 4, 256, 128
    ctx = 1000
    g = torch.Generator().manual_seed(77)
    u = torch.randn(hkv, d, generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    ramp = torch.arange(ctx, dtype=torch.float32) / 64.0
    if order == "falling":
        ramp = ramp.flip(0)
    nb = math.ceil(ctx / bs) + 2
    key = torch.zeros(nb * bs, hkv, d)
    key[:ctx] = ramp[:, None, None] * u[None] + 0.05 * torch.randn(ctx, hkv, d, generator=g)
    value = torch.randn(nb * bs, hkv, d, generator=g)
    key, value = key.to(torch.bfloat16), value.to(torch.bfloat16)
    ks = (key.float().abs().amax(dim=(0, 2)) / o.MAX_FINITE).to(device)
    vs = (value.float().abs().amax(dim=(0, 2)) / o.MAX_FINITE).to(device)
    kc = torch.zeros((nb, bs, hkv, d + 4), dtype=torch.uint8, device=device)
    vc = torch.zeros((nb, bs, hkv, d + 4), dtype=torch.uint8, device=device)
    kv_cache.write_kv_cache(key.to(device), value.to(device), kc, vc, torch.arange(nb * bs, device=device), ks, vs)
    table = torch.randperm(nb, generator=g)[None, :].to(torch.int32)
    # q along u with |q| so that one tile (64 keys, ramp + 1) adds ~16 log2 units to the logit.
    q = (u.repeat_interleave(hq // hkv, dim=0)[None] * (16.0 / math.log2(math.e)) * math.sqrt(d)
         + 0.1 * torch.randn(qlen, hq, d, generator=g)).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(d)
    print(f"case growing max order={order} qlen={qlen}", flush=True)
    out = _run_op(device, q, kc, vc, table, [ctx], [qlen], scale, True)
    got = out.float().cpu().numpy()
    ref = o.paged_attention_reference(q.float().numpy(), kc.cpu().numpy(), vc.cpu().numpy(), table.numpy(), [ctx],
                                      bs, scale, rounding="f64", query_lens=[qlen], causal=True, dtype="bf16")
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2)


def test_prefill_fp16_query(native_ops, device):
    _check(device, [600, 130], [70, 130], 16, 4, 256, 128, dtype=torch.float16, seed=20)


@pytest.mark.parametrize("hq,hkv,d,bs,lens,qlens,bt_dtype", [
    (8, 2, 128, 16, [45, 300, 47], [45, 20, 1], torch.int64),   # block size 16: tiles span pages
    (16, 1, 64, 32, [100, 64], [37, 64], torch.int32),           # group 16: 4 tokens per tile
    (8, 8, 128, 64, [70, 200], [70, 3], torch.int64),            # group 1: 64 tokens per tile
    (16, 4, 256, 48, [200, 97], [66, 97], torch.int32),          # block size 48 (not a power of two)
    (4, 2, 64, 128, [1000], [130], torch.int32),                 # group 2
    (16, 2, 128, 128, [513], [300], torch.int32),                # group 8
])
def test_prefill_other_shapes(native_ops, device, hq, hkv, d, bs, lens, qlens, bt_dtype):
    _check(device, lens, qlens, hq, hkv, d, bs, bt_dtype=bt_dtype, seed=hq + d + bs)


@pytest.mark.parametrize("hq,hkv,d,dv,bs,lens,qlens", [
    (4, 2, 24, 24, 4, [9, 3, 0], [4, 3, 0]),     # head size outside the MFMA set
    (4, 2, 64, 32, 8, [40, 17], [12, 2]),        # head_size_v != head_size
    (20, 1, 64, 64, 16, [33], [33]),             # group 20 > 16
    (12, 4, 64, 64, 16, [50, 20], [7, 20]),      # group 3, not a power of two
])
def test_prefill_any_shape_kernel(native_ops, device, hq, hkv, d, dv, bs, lens, qlens):
    _check(device, lens, qlens, hq, hkv, d, bs, dv=dv, seed=d + dv + hq)


def test_prefill_mixed_chunked_batch(native_ops, device):
    """A chunked-prefill step: decode rows (one token) beside long chunks and
    short ones.  Only the long requests (more than 128 (token, head) rows:
    200, 40 and 50 tokens at G = 4) get tile images; the decode rows and the
    17-token chunk run the in-kernel page decode in the same call, in
    whatever order the batch lists them."""
    _check(device, [900, 2000, 600, 4096, 700, 50], [1, 200, 17, 1, 40, 50], 16, 4, 256, 128, seed=25)
    _check(device, [4096, 900, 3000], [300, 1, 1], 16, 4, 256, 128, seed=26)


def test_prefill_long_requests_past_the_image_slots(native_ops, device, monkeypatch):
    """With the image budget capped at 1 MiB only one long request gets a slot
    (at least one always does); the other long requests run the in-kernel
    path, which then covers all of their query tiles."""
    monkeypatch.setenv("HIF8_PREFILL_IMAGE_CAP_MB", "1")
    _check(device, [600, 300, 640, 90, 500], [100, 1, 64, 90, 33], 16, 4, 256, 128, seed=27)
    monkeypatch.setenv("HIF8_PREFILL_IMAGE_CAP_MB", "0")
    _check(device, [1000, 700], [70, 700], 16, 4, 256, 128, seed=28)


def test_prefill_is_deterministic(native_ops, device):
    # 30 rows: the in-kernel page decode; 100 rows: tile images, with key splits.
    kc, vc, table = build_cache(device, [4096], 4, 256, 128, 21)
    for rows in (30, 100):
        q = randn((rows, 16, 256), 22)
        a = _run_op(device, q, kc, vc, table, [4096], [rows], 0.0625, True)
        b = _run_op(device, q, kc, vc, table, [4096], [rows], 0.0625, True)
        assert torch.equal(a, b), rows


def test_prefill_api_validation(native_ops, device):
    from hif8_rocm import kv_cache

    kc, vc, table = build_cache(device, [100], 4, 256, 128, 23)
    q = randn((10, 16, 256), 24).to(device)
    with pytest.raises(ValueError, match="describe every query row"):
        kv_cache.paged_attention(q, kc, vc, table.to(device), [100], scale=0.0625, query_lens=[9])
    with pytest.raises(ValueError, match="cannot be shorter"):
        kv_cache.paged_attention(q, kc, vc, table.to(device), [5], scale=0.0625, query_lens=[10])
    bad = table.clone()
    bad[0, 0] = kc.shape[0] + 3
    with pytest.raises(IndexError, match="outside the cache"):
        kv_cache.paged_attention(q, kc, vc, bad.to(device), [100], scale=0.0625, query_lens=[10])
