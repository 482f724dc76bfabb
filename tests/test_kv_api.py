"""Host-side KV cache API (CPU): the layout mirrors the reference's
Hif8KVCacheLayout (kv_cache.py:26-88; test_hif8_kv_cache.py:74-92), pack and
unpack match the oracle byte for byte, the new operators have Meta shapes, and
the C ABI validates arguments and sizes its workspace without a GPU."""

import ctypes

import numpy as np
import pytest
import torch

from conftest import PKG_ROOT
from hif8_rocm import kv_cache, native
from oracle import hif8_oracle as o


def test_layout_accounts_for_k_and_v_inline_scales():
    layout = kv_cache.Hif8KVCacheLayout(3, 8, 2, 16, 24)
    assert layout.key_width == 20 and layout.value_width == 28
    assert layout.page_size_bytes == 8 * 2 * (20 + 28)
    assert layout.key_shape() == (3, 8, 2, 20) and layout.value_shape() == (3, 8, 2, 28)
    qwen = kv_cache.Hif8KVCacheLayout(1, 128, 4, 256)
    assert qwen.resolved_head_size_v == 256 and qwen.key_page_size_bytes == 128 * 4 * 260 == 133120
    k, v = qwen.allocate("cpu")
    assert k.shape == (1, 128, 4, 260) and v.dtype == torch.uint8 and not k.any()


@pytest.mark.parametrize("args", [(0, 8, 2, 16), (1, 8, 2, 18), (1, 8, 2, 16, 10), (1, 8, 2.0, 16)])
def test_invalid_layout_dimensions_are_rejected(args):
    with pytest.raises(ValueError):
        kv_cache.Hif8KVCacheLayout(*args)


def test_pack_unpack_match_the_oracle():
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 256, (5, 3, 12), dtype=np.uint8)
    scale = rng.random((5, 3)).astype(np.float32)
    packed = kv_cache.pack_kv_rows(torch.from_numpy(codes), torch.from_numpy(scale))
    assert np.array_equal(packed.numpy(), o.pack_kv_rows(codes, scale))
    data, back = kv_cache.unpack_kv_rows(packed, 12)
    assert np.array_equal(data.numpy(), codes) and np.array_equal(back.numpy(), scale)
    with pytest.raises(TypeError):
        kv_cache.pack_kv_rows(torch.from_numpy(codes), torch.from_numpy(scale).double())
    with pytest.raises(ValueError):
        kv_cache.unpack_kv_rows(packed, 8)


def test_kv_operator_meta_shapes():
    native.load_extension()
    q = torch.empty(3, 16, 256, dtype=torch.bfloat16, device="meta")
    kc = torch.empty(10, 128, 4, 260, dtype=torch.uint8, device="meta")
    vc = torch.empty(10, 128, 4, 132, dtype=torch.uint8, device="meta")
    out = torch.ops.vllm_ascend_hif8.hif8_paged_decode_attention(
        q, kc, vc, torch.empty(3, 4, dtype=torch.int32, device="meta"),
        torch.empty(3, dtype=torch.int32, device="meta"), 0.0625, 500)
    assert out.shape == (3, 16, 128) and out.dtype == torch.bfloat16


def test_write_and_attention_reject_bad_arguments_before_launch():
    kc = torch.zeros(2, 4, 2, 20, dtype=torch.uint8)
    vc = torch.zeros(2, 4, 2, 20, dtype=torch.uint8)
    key = torch.zeros(3, 2, 16, dtype=torch.bfloat16)
    ones = torch.ones(2)
    with pytest.raises(IndexError, match="invalid block"):
        kv_cache.write_kv_cache(key, key, kc, vc, torch.tensor([0, 8, -1]), ones, ones)
    with pytest.raises(ValueError, match="do not match"):
        kv_cache.write_kv_cache(key[..., :12], key, kc, vc, torch.tensor([0, 1, 2]), ones, ones)
    with pytest.raises(ValueError, match="num_actual_tokens"):
        kv_cache.write_kv_cache(key, key, kc, vc, torch.tensor([0, 1, 2]), ones, ones, num_actual_tokens=4)
    q = torch.zeros(1, 4, 16, dtype=torch.bfloat16)
    table = torch.tensor([[1, 5]])
    with pytest.raises(IndexError, match="outside the cache"):
        kv_cache.paged_decode_attention(q, kc, vc, table, [6], scale=0.25)
    with pytest.raises(ValueError, match="too few entries"):
        kv_cache.paged_decode_attention(q, kc, vc, table, [9], scale=0.25)
    with pytest.raises(ValueError, match="divisible"):
        kv_cache.paged_decode_attention(torch.zeros(1, 3, 16, dtype=torch.bfloat16), kc, vc, table, [2], scale=0.25)
    # A caller-supplied max_query_len below the longest request is caught by validation.
    q3 = torch.zeros(5, 4, 16, dtype=torch.bfloat16)
    loc = torch.tensor([0, 2, 5], dtype=torch.int32)
    with pytest.raises(ValueError, match="max_query_len"):
        kv_cache.paged_attention(q3, kc, vc, torch.tensor([[0], [1]]), [3, 4], scale=0.25, query_start_loc=loc,
                                 max_query_len=2)


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(str(PKG_ROOT / "hif8_rocm" / "libhif8_rocm.so"))
    lib.hif8_last_error.restype = ctypes.c_char_p
    return lib


def test_workspace_size_follows_the_split_plan(lib):
    f = lib.hif8_paged_decode_attention_workspace_size
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_int64] * 6
    # One request of 16384 tokens = 512 tiles x 4 KV heads: 4 tiles per split keeps
    # 512 workgroups -> 128 splits x 16 heads x (256 + 2) floats.
    assert f(1, 16, 4, 256, 256, 16384) == 128 * 16 * 258 * 4
    # Batch 4: at most 8 tiles per split -> 64 splits per request.
    assert f(4, 16, 4, 256, 256, 16384) == 4 * 64 * 16 * 258 * 4
    # Batch 1, 4096 tokens: 512 workgroups with one tile each -> 128 splits.
    assert f(1, 16, 4, 256, 256, 4096) == 128 * 16 * 258 * 4
    assert f(1, 16, 4, 256, 256, 32) == 0          # a single split needs no workspace
    assert f(1, 16, 4, 24, 24, 4096) == 0          # any-shape kernel
    assert f(1, 15, 4, 256, 256, 4096) == 0        # heads not divisible


def test_kv_entry_points_validate_arguments(lib):
    P, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    w = lib.hif8_kv_cache_write
    w.argtypes = [P, P, I, L, L, L, L, P, P, P, I, P, P, L, L, P, P]
    p = ctypes.c_void_p(16)
    assert w(p, p, 1, 4, 4, 18, 18, p, p, p, 1, p, p, 2, 128, None, None) == 1
    assert b"divisible by four" in lib.hif8_last_error()
    assert w(p, p, 1, 4, 4, 256, 256, p, p, p, 7, p, p, 2, 128, None, None) == 1
    assert b"int32 or int64" in lib.hif8_last_error()
    assert w(None, p, 1, 4, 4, 256, 256, p, p, p, 1, p, p, 2, 128, None, None) == 1
    assert b"null pointer" in lib.hif8_last_error()
    assert w(None, None, 1, 0, 4, 256, 256, None, None, None, 1, None, None, 2, 128, None, None) == 0
    a = lib.hif8_paged_decode_attention
    a.argtypes = [P, I, P, P, L, L, L, L, L, P, I, L, P, L, L, L, ctypes.c_float, P, P, ctypes.c_size_t, P]
    assert a(p, 1, p, p, 8, 128, 4, 256, 256, p, 0, 4, p, 2, 15, 512, 0.0625, p, None, 0, None) == 1
    assert b"divisible by num_kv_heads" in lib.hif8_last_error()
    assert a(p, 1, p, p, 8, 128, 4, 256, 256, p, 0, 4, p, 2, 16, 513, 0.0625, p, None, 0, None) == 1
    assert b"block table capacity" in lib.hif8_last_error()
    assert a(p, 1, p, p, 8, 128, 4, 256, 256, p, 0, 4, p, 2, 16, 512, 0.0625, p, None, 0, None) == 1
    assert b"workspace" in lib.hif8_last_error()
