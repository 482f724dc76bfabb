"""Pins the oracle's KV functions (CPU): byte layout, slot scatter and page
gather against the reference's known answers (test_hif8_kv_cache.py:74-197),
static KV quant against the static codec with per-head scales
(test_hif8_kv_npu.py:380-551), and paged attention against closed forms, a
head-mapping check and a per-token loop."""

import math
import struct

import numpy as np
import pytest

from oracle import hif8_oracle as o

KEY_SCALES_L3 = np.array([0.9432383179664612, 0.7343872785568237, 0.9391698241233826, 1.1160656213760376], np.float32)


def test_pack_unpack_is_byte_exact():
    codes = np.array([[[o.encode_scalar(v) for v in (-1.0, 0.5, 0.0, 1.0)],
                       [o.encode_scalar(v) for v in (0.25, -0.25, 0.75, -0.75)]]], np.uint8)
    scale = np.array([[2.0, 3.0]], np.float32)
    packed = o.pack_kv_rows(codes, scale)
    assert packed.shape == (1, 2, 8) and packed.dtype == np.uint8
    # Codes first, then the scale's IEEE-754 bytes, little-endian: 2.0 = 0x40000000, 3.0 = 0x40400000.
    assert list(packed[0, 0, 4:]) == [0x00, 0x00, 0x00, 0x40]
    assert list(packed[0, 1, 4:]) == [0x00, 0x00, 0x40, 0x40]
    assert list(packed[0, 0, :4]) == [0x88, 0x18, 0x00, 0x08]
    data, back = o.unpack_kv_rows(packed, 4)
    assert np.array_equal(data, codes) and np.array_equal(back, scale)
    with pytest.raises(ValueError):
        o.unpack_kv_rows(packed, 5)


def test_slot_mapping_and_block_table_gather():
    cache = np.zeros((2, 4, 1, 8), np.uint8)
    rows = np.arange(24, dtype=np.uint8).reshape(3, 1, 8)
    o.scatter_kv_rows(cache, rows, np.array([0, 5, -1]), block_size=4)
    got = o.gather_kv_rows(cache, np.array([[0, 1]]), [6], block_size=4)[0]
    assert np.array_equal(got[0], rows[0]) and np.array_equal(got[5], rows[1])
    assert not got[1].any() and not got[2].any()
    with pytest.raises(IndexError):
        o.scatter_kv_rows(cache, rows, np.array([0, 8, -1]), block_size=4)


def test_concat_gather_follows_the_slot_formula():
    cache = (np.arange(5 * 4 * 2 * 8) % 256).astype(np.uint8).reshape(5, 4, 2, 8)
    table = np.array([[3, 1, -1], [4, 0, 2]])
    got = o.gather_kv_rows_concat(cache, table, [5, 10], block_size=4)
    flat = cache.reshape(-1, 2, 8)
    want = [flat[table[b, t // 4] * 4 + t % 4] for b, n in ((0, 5), (1, 10)) for t in range(n)]
    assert np.array_equal(got, np.stack(want))
    zero = o.gather_kv_rows_concat(cache[:2], np.array([[-1], [1]]), [0, 3], block_size=4)
    assert np.array_equal(zero, cache[1, :3])
    with pytest.raises(IndexError):
        o.gather_kv_rows(cache, np.array([[7]]), [2], block_size=4)


def test_static_kv_quant_uses_the_head_scale_of_each_row():
    rng = np.random.default_rng(20260822)
    x = (rng.standard_normal((9, 4, 32)) * 3.0).astype(np.float32)
    data, row_scale = o.quantize_kv_rows_static(x, KEY_SCALES_L3)
    assert np.array_equal(row_scale, np.broadcast_to(KEY_SCALES_L3, (9, 4)))
    for h in range(4):
        want = np.array([[o.encode_scalar(float(np.clip(np.float32(v) / KEY_SCALES_L3[h], -2.0 ** 15, 2.0 ** 15)))
                          for v in row] for row in x[:, h]], np.uint8)
        assert np.array_equal(data[:, h], want)


def _cache_from_values(values, scales):
    """[T, H, D] float values that are exact HiF8 multiples of per-head scales -> packed rows."""
    data, row_scale = o.quantize_kv_rows_static(values, scales)
    return o.pack_kv_rows(data, row_scale)


def test_attention_closed_form():
    # kv_cache reference test: keys alternate e0/e1, values 2*e0 / 3*e1.
    key = np.array([[[1, 0, 0, 0]], [[0, 1, 0, 0]], [[1, 0, 0, 0]], [[0, 1, 0, 0]]], np.float32)
    value = np.array([[[2, 0, 0, 0]], [[0, 3, 0, 0]], [[2, 0, 0, 0]], [[0, 3, 0, 0]]], np.float32)
    kc = _cache_from_values(key, np.array([1.0], np.float32)).reshape(1, 4, 1, 8)
    vc = _cache_from_values(value, np.array([1.0], np.float32)).reshape(1, 4, 1, 8)
    q = np.array([[[1.0, 0.0, 0.0, 0.0]]], np.float32)
    out = o.paged_attention_reference(q, kc, vc, np.array([[0]]), [4], block_size=4, scale=1.0, rounding="f64")
    z = 2 * math.e + 2
    assert np.allclose(out[0, 0], [2 * 2 * math.e / z, 3 * 2 / z, 0, 0], rtol=0, atol=1e-12)
    bf = o.paged_attention_reference(q, kc, vc, np.array([[0]]), [4], block_size=4, scale=1.0, rounding="bf16")
    assert np.allclose(bf, out, rtol=2 ** -7, atol=0)
    assert bf[0, 0, 0] > 1.0 and bf[0, 0, 1] < 2.0


def test_attention_maps_query_head_h_to_kv_head_h_over_group():
    # Constant values per KV head: the output of query head h is exactly the
    # value of the KV head it attends (softmax weights sum to one).
    hkv, group, d, t = 2, 3, 8, 5
    rng = np.random.default_rng(3)
    key = rng.integers(-4, 5, (t, hkv, d)).astype(np.float32)
    value = np.empty((t, hkv, d), np.float32)
    value[:, 0] = 1.0
    value[:, 1] = 2.0
    kc = _cache_from_values(key, np.ones(hkv, np.float32)).reshape(1, t, hkv, d + 4)
    vc = _cache_from_values(value, np.ones(hkv, np.float32)).reshape(1, t, hkv, d + 4)
    q = rng.standard_normal((1, hkv * group, d)).astype(np.float32)
    out = o.paged_attention_reference(q, kc, vc, np.array([[0]]), [t], block_size=t, scale=0.5, rounding="f64")
    assert np.allclose(out[0, :, 0], [1, 1, 1, 2, 2, 2], rtol=0, atol=1e-12)


def _bf16(x: float) -> float:
    return float(o.round_bf16(np.array([x], np.float32))[0])


def _f16(x: float) -> float:
    """IEEE half, round to nearest even, by the struct module (no numpy)."""
    return struct.unpack("<e", struct.pack("<e", float(x)))[0]


def test_attention_matches_per_token_loop_and_empty_requests():
    rng = np.random.default_rng(5)
    hkv, group, d, bs, nb = 2, 2, 8, 4, 6
    kc = np.zeros((nb, bs, hkv, d + 4), np.uint8)
    vc = np.zeros_like(kc)
    kvals = rng.standard_normal((nb * bs, hkv, d)).astype(np.float32)
    vvals = rng.standard_normal((nb * bs, hkv, d)).astype(np.float32)
    ks, vs = np.array([0.01, 0.02], np.float32), np.array([0.03, 0.005], np.float32)
    o.scatter_kv_rows(kc, _cache_from_values(kvals, ks), np.arange(nb * bs), bs)
    o.scatter_kv_rows(vc, _cache_from_values(vvals, vs), np.arange(nb * bs), bs)
    table = np.array([[5, 2, -1], [0, 1, 3], [4, -1, -1]])
    lens = [6, 11, 0]
    q = rng.standard_normal((3, hkv * group, d)).astype(np.float32)
    out = o.paged_attention_reference(q, kc, vc, table, lens, block_size=bs, scale=0.3, rounding="f64")
    for b, n in enumerate(lens):
        for h in range(hkv * group):
            j = h // group
            logits, rows = [], []
            for t in range(n):
                slot = table[b, t // bs] * bs + t % bs
                kd, ksc = o.unpack_kv_rows(kc.reshape(-1, hkv, d + 4)[slot:slot + 1], d)
                vd, vsc = o.unpack_kv_rows(vc.reshape(-1, hkv, d + 4)[slot:slot + 1], d)
                k = [_bf16(o.decode_scalar(int(c)) * ksc[0, j]) for c in kd[0, j]]
                v = [_bf16(o.decode_scalar(int(c)) * vsc[0, j]) for c in vd[0, j]]
                logits.append(0.3 * sum(float(a) * b_ for a, b_ in zip(q[b, h], k)))
                rows.append(v)
            if not n:
                assert not out[b, h].any()
                continue
            m = max(logits)
            w = [math.exp(x - m) for x in logits]
            want = [sum(wi * r[i] for wi, r in zip(w, rows)) / sum(w) for i in range(d)]
            assert np.allclose(out[b, h], want, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- multi-token (prefill / chunked prefill)

def _attention_loop(query, kc, vc, table, lens, bs, scale, query_lens, causal, kv_round=_bf16):
    """Per query row and head, keys walked through the block table one token
    at a time and the softmax written out by hand (no array code shared with
    the oracle): query row i of request b sits at position lens[b] -
    query_lens[b] + i (kv_cache.py:365-369)."""
    hq, d = query.shape[1], query.shape[2]
    hkv = kc.shape[2]
    group = hq // hkv
    flat_k, flat_v = kc.reshape(-1, hkv, d + 4), vc.reshape(-1, hkv, d + 4)
    out, r = [], 0
    for b, (ql, kl) in enumerate(zip(query_lens, lens)):
        for i in range(ql):
            last = kl - ql + i if causal else kl - 1
            heads = []
            for h in range(hq):
                j = h // group
                logits, rows = [], []
                for t in range(min(last + 1, kl)):
                    slot = table[b, t // bs] * bs + t % bs
                    kd, ksc = o.unpack_kv_rows(flat_k[slot:slot + 1], d)
                    vd, vsc = o.unpack_kv_rows(flat_v[slot:slot + 1], d)
                    k = [kv_round(o.decode_scalar(int(c)) * ksc[0, j]) for c in kd[0, j]]
                    rows.append([kv_round(o.decode_scalar(int(c)) * vsc[0, j]) for c in vd[0, j]])
                    logits.append(scale * sum(float(a) * b_ for a, b_ in zip(query[r, h], k)))
                if not logits:
                    heads.append([0.0] * d)
                    continue
                m = max(logits)
                w = [math.exp(x - m) for x in logits]
                heads.append([sum(wi * row[x] for wi, row in zip(w, rows)) / sum(w) for x in range(d)])
            out.append(heads)
            r += 1
    return np.asarray(out, np.float64).reshape(r, hq, d)


def _random_paged_cache(rng, nb, bs, hkv, d):
    kc = np.zeros((nb, bs, hkv, d + 4), np.uint8)
    vc = np.zeros_like(kc)
    kvals = rng.standard_normal((nb * bs, hkv, d)).astype(np.float32)
    vvals = rng.standard_normal((nb * bs, hkv, d)).astype(np.float32)
    ks = (np.abs(kvals).max(axis=(0, 2)) / 32768.0).astype(np.float32)
    vs = (np.abs(vvals).max(axis=(0, 2)) / 32768.0).astype(np.float32)
    o.scatter_kv_rows(kc, _cache_from_values(kvals, ks), np.arange(nb * bs), bs)
    o.scatter_kv_rows(vc, _cache_from_values(vvals, vs), np.arange(nb * bs), bs)
    return kc, vc


@pytest.mark.parametrize("causal", [True, False])
def test_multi_token_attention_matches_per_row_loop(causal):
    rng = np.random.default_rng(17)
    hkv, group, d, bs, nb = 2, 2, 8, 4, 8
    kc, vc = _random_paged_cache(rng, nb, bs, hkv, d)
    table = np.array([[6, 1, 3, -1], [0, 7, 2, 5], [4, -1, -1, -1], [-1, -1, -1, -1]])
    lens, qlens = [9, 14, 3, 0], [4, 14, 1, 0]
    q = rng.standard_normal((sum(qlens), hkv * group, d)).astype(np.float32)
    out = o.paged_attention_reference(q, kc, vc, table, lens, bs, 0.35, rounding="f64", query_lens=qlens,
                                      causal=causal)
    want = _attention_loop(q, kc, vc, table, lens, bs, 0.35, qlens, causal)
    assert out.shape == (sum(qlens), hkv * group, d)
    assert np.allclose(out, want, rtol=1e-12, atol=1e-12)
    bf = o.paged_attention_reference(q, kc, vc, table, lens, bs, 0.35, rounding="bf16", query_lens=qlens,
                                     causal=causal)
    assert np.allclose(bf, out, rtol=0, atol=3e-2)


def test_fp16_queries_round_kv_and_intermediates_to_fp16():
    """dtype="f16": K/V rows rounded to fp16 (decode_kv_rows(...).to(query.dtype),
    kv_cache.py:355-356), checked against the per-row loop with a struct-module
    fp16 rounding; the query-dtype intermediates stay within fp16 resolution of
    the float64 path, and differ from the bf16 ones."""
    rng = np.random.default_rng(23)
    hkv, group, d, bs, nb = 2, 2, 8, 4, 8
    kc, vc = _random_paged_cache(rng, nb, bs, hkv, d)
    table = np.array([[6, 1, 3, -1], [0, 7, 2, 5]])
    lens, qlens = [9, 14], [4, 3]
    q = rng.standard_normal((sum(qlens), hkv * group, d)).astype(np.float32)
    f64 = o.paged_attention_reference(q, kc, vc, table, lens, bs, 0.35, rounding="f64", query_lens=qlens,
                                      dtype="f16")
    want = _attention_loop(q, kc, vc, table, lens, bs, 0.35, qlens, True, kv_round=_f16)
    assert np.allclose(f64, want, rtol=1e-12, atol=1e-12)
    b16 = o.paged_attention_reference(q, kc, vc, table, lens, bs, 0.35, rounding="f64", query_lens=qlens)
    assert not np.allclose(f64, b16, rtol=1e-9, atol=1e-9)
    r16 = o.paged_attention_reference(q, kc, vc, table, lens, bs, 0.35, rounding="bf16", query_lens=qlens,
                                      dtype="f16")
    assert np.allclose(r16, f64, rtol=0, atol=4e-3)
    assert np.array_equal(r16, r16.astype(np.float16).astype(np.float64))   # outputs are fp16 values
    with pytest.raises(ValueError, match="dtype"):
        o.paged_attention_reference(q, kc, vc, table, lens, bs, 0.35, query_lens=qlens, dtype="fp8")


def test_right_aligned_causal_mask_closed_form():
    # Zero keys make every visible logit equal, so each output is the mean of
    # the values the row may see.  Value row t is the constant t + 1 (exact in
    # HiF8), so row i of a request with L cached tokens and q query rows sees
    # positions 0 .. L - q + i and outputs (L - q + i + 2) / 2.  A mask
    # aligned to the top-left (row i sees 0 .. i) would give (i + 2) / 2.
    bs, d, hkv = 4, 4, 1
    lens, qlens = [11, 6], [5, 6]
    nb = 5
    kc = _cache_from_values(np.zeros((nb * bs, hkv, d), np.float32), np.ones(1, np.float32)).reshape(nb, bs, hkv, d + 4)
    vc = np.zeros_like(kc)
    table = np.array([[2, 0, 4], [1, 3, -1]])
    # Write value t + 1 at token t of each request.
    for b, n in enumerate(lens):
        for t in range(n):
            slot = table[b, t // bs] * bs + t % bs
            row = _cache_from_values(np.full((1, hkv, d), t + 1, np.float32), np.ones(1, np.float32))
            vc.reshape(-1, hkv, d + 4)[slot] = row[0]
    q = np.ones((sum(qlens), 2, d), np.float32)
    out = o.paged_attention_reference(q, kc, vc, table, lens, bs, 1.0, rounding="f64", query_lens=qlens)
    r = 0
    for n, ql in zip(lens, qlens):
        for i in range(ql):
            right = (n - ql + i + 2) / 2.0
            assert np.allclose(out[r], right, rtol=0, atol=1e-12), (n, ql, i)
            if n != ql:
                assert not np.allclose(out[r], (i + 2) / 2.0)
            r += 1
    # Without the mask every row sees the whole request: mean of 1 .. L.
    full = o.paged_attention_reference(q, kc, vc, table, lens, bs, 1.0, rounding="f64", query_lens=qlens,
                                       causal=False)
    assert np.allclose(full[:5], (lens[0] + 1) / 2.0) and np.allclose(full[5:], (lens[1] + 1) / 2.0)


def test_one_query_row_per_request_is_the_decode_case():
    rng = np.random.default_rng(23)
    hkv, group, d, bs, nb = 2, 4, 8, 4, 6
    kc, vc = _random_paged_cache(rng, nb, bs, hkv, d)
    table = np.array([[5, 2, 0], [1, 3, 4]])
    lens = [7, 12]
    q = rng.standard_normal((2, hkv * group, d)).astype(np.float32)
    for rounding in ("f64", "bf16"):
        dec = o.paged_attention_reference(q, kc, vc, table, lens, bs, 0.5, rounding=rounding)
        pre = o.paged_attention_reference(q, kc, vc, table, lens, bs, 0.5, rounding=rounding, query_lens=[1, 1])
        assert np.array_equal(dec, pre)


def test_rows_before_the_first_key_are_zero_and_lengths_are_checked():
    rng = np.random.default_rng(29)
    kc, vc = _random_paged_cache(rng, 2, 4, 1, 4)
    q = rng.standard_normal((5, 1, 4)).astype(np.float32)
    # Five query rows over three cached tokens: rows 0 and 1 sit at negative
    # positions and see nothing.
    out = o.paged_attention_reference(q, kc, vc, np.array([[1]]), [3], 4, 1.0, rounding="f64", query_lens=[5])
    assert not out[:2].any() and np.abs(out[2:]).sum() > 0
    with pytest.raises(ValueError):
        o.paged_attention_reference(q, kc, vc, np.array([[1]]), [3], 4, 1.0, query_lens=[4])
