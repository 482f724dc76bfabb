"""hif8_paged_decode_attention_noalloc through the C ABI (ctypes, raw device
pointers) against hif8_paged_decode_attention with a caller workspace: the
same kernels and split plan, so the outputs are equal bit for bit.  Two calls
in a row, the second with a smaller input (the shared scratch array keeps the
first call's partials, which the second must not read), then the first size
again; the first call made under HIP graph capture and replayed; sizes whose
partials exceed the scratch array are rejected before any launch; a size
without splits needs no scratch."""

import ctypes
import math

import pytest
import torch

from _kv import build_cache, randn
from conftest import PKG_ROOT

pytestmark = pytest.mark.gpu
LIB = PKG_ROOT / "hif8_rocm" / "libhif8_rocm.so"
BF16, INT32 = 1, 0
SCRATCH_BYTES = 16 << 20


@pytest.fixture(scope="module")
def lib(native_ops):
    lib = ctypes.CDLL(str(LIB))
    lib.hif8_last_error.restype = ctypes.c_char_p
    common = ([ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 5 +
              [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p] + [ctypes.c_int64] * 3 +
              [ctypes.c_float, ctypes.c_void_p])
    lib.hif8_paged_decode_attention.argtypes = common + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.hif8_paged_decode_attention_noalloc.argtypes = common + [ctypes.c_void_p]
    lib.hif8_paged_decode_attention_workspace_size.argtypes = [ctypes.c_int64] * 6
    lib.hif8_paged_decode_attention_workspace_size.restype = ctypes.c_size_t
    return lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _case(device, lens, seed):
    kc, vc, table = build_cache(device, lens, 4, 256, 128, seed, bt_dtype=torch.int32)
    q = randn((len(lens), 16, 256), seed + 1).to(device)
    return kc, vc, table.to(device), q, torch.tensor(lens, dtype=torch.int32, device=device)


def _args(kc, vc, table, q, lens_dev, max_len, out):
    return [_ptr(q), BF16, _ptr(kc), _ptr(vc), kc.shape[0], kc.shape[1], 4, 256, 256, _ptr(table), INT32,
            table.shape[1], _ptr(lens_dev), q.shape[0], 16, max_len, 1.0 / math.sqrt(256), _ptr(out)]


def _run_both(lib, device, lens, seed):
    kc, vc, table, q, lens_dev = _case(device, lens, seed)
    max_len = max(lens)
    need = lib.hif8_paged_decode_attention_workspace_size(len(lens), 16, 4, 256, 256, max_len)
    print(f"noalloc case lens={lens} workspace={need}", flush=True)
    assert 0 < need <= SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    want = torch.empty(len(lens), 16, 256, dtype=torch.bfloat16, device=device)
    got = torch.full_like(want, float("nan"))
    torch.cuda.synchronize()
    assert lib.hif8_paged_decode_attention(*_args(kc, vc, table, q, lens_dev, max_len, want), _ptr(ws), need,
                                           None) == 0, lib.hif8_last_error()
    assert lib.hif8_paged_decode_attention_noalloc(*_args(kc, vc, table, q, lens_dev, max_len, got),
                                                   None) == 0, lib.hif8_last_error()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    return got


def test_noalloc_first_call_captured_in_a_graph(lib, device):
    """The process's first call of the entry point (defined first here; no other
    test calls it) is made under HIP graph capture, so the scratch address is
    resolved inside the capture.  The graph is replayed three times with eager
    work in between - a smaller eager call that overwrites the shared scratch,
    and the output reset - and every replay equals the workspace entry point
    bit for bit."""
    kc, vc, table, q, lens_dev = _case(device, [16384, 3000, 700], 44)
    max_len = 16384
    need = lib.hif8_paged_decode_attention_workspace_size(3, 16, 4, 256, 256, max_len)
    assert 0 < need <= SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=device)
    want = torch.empty(3, 16, 256, dtype=torch.bfloat16, device=device)
    got = torch.full_like(want, float("nan"))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.hif8_paged_decode_attention(*_args(kc, vc, table, q, lens_dev, max_len, want), _ptr(ws), need,
                                           stream) == 0, lib.hif8_last_error()
    torch.cuda.synchronize()
    print("noalloc capture: recording the first call", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        st = lib.hif8_paged_decode_attention_noalloc(*_args(kc, vc, table, q, lens_dev, max_len, got), cap)
    assert st == 0, lib.hif8_last_error()
    other = _case(device, [5000, 64], 45)
    other_out = torch.empty(2, 16, 256, dtype=torch.bfloat16, device=device)
    for rep in range(3):
        got.fill_(float("nan"))
        assert lib.hif8_paged_decode_attention_noalloc(*_args(*other, 5000, other_out), stream) == 0
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"noalloc capture: replay {rep}", flush=True)
        assert torch.equal(got, want), rep


def test_noalloc_matches_the_workspace_entry_point_twice_then_smaller(lib, device):
    big = _run_both(lib, device, [16384, 9000, 4096, 16384], 41)        # 8.5 MB of partials
    small = _run_both(lib, device, [700, 3000], 42)                     # fewer splits, stale partials above
    again = _run_both(lib, device, [16384, 9000, 4096, 16384], 41)
    assert torch.equal(big, again) and small.shape[0] == 2


def test_noalloc_rejects_sizes_beyond_the_scratch_array(lib, device):
    need = lib.hif8_paged_decode_attention_workspace_size(64, 16, 4, 256, 256, 16384)
    assert need > SCRATCH_BYTES
    dummy = torch.empty(16, dtype=torch.uint8, device=device)
    p = _ptr(dummy)
    st = lib.hif8_paged_decode_attention_noalloc(p, BF16, p, p, 8192, 128, 4, 256, 256, p, INT32, 128, p, 64, 16,
                                                 16384, 0.0625, p, None)
    assert st == 2 and b"scratch array" in lib.hif8_last_error()


def test_noalloc_without_splits_needs_no_scratch(lib, device):
    # A context of one 32-token tile runs as a single split.
    kc, vc, table, q, lens_dev = _case(device, [30], 43)
    assert lib.hif8_paged_decode_attention_workspace_size(1, 16, 4, 256, 256, 30) == 0
    want = torch.empty(1, 16, 256, dtype=torch.bfloat16, device=device)
    got = torch.full_like(want, float("nan"))
    assert lib.hif8_paged_decode_attention(*_args(kc, vc, table, q, lens_dev, 30, want), None, 0, None) == 0
    assert lib.hif8_paged_decode_attention_noalloc(*_args(kc, vc, table, q, lens_dev, 30, got), None) == 0
    torch.cuda.synchronize()
    assert torch.equal(got, want)
