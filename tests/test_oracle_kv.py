"""Pins the oracle's KV functions (CPU): byte layout, slot scatter and page
gather against the reference's known answers (test_hif8_kv_cache.py:74-197),
static KV quant against the static codec with per-head scales
(test_hif8_kv_npu.py:380-551), and paged attention against closed forms, a
head-mapping check and a per-token loop."""

import math

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
