"""The C-ABI library loads without a GPU, exports every function declared in
include/*.h and rejects invalid arguments before touching the device (CPU)."""

import ctypes
import re

import pytest

from conftest import PKG_ROOT, REPO

LIB = PKG_ROOT / "hif8_rocm" / "libhif8_rocm.so"


def _declared_functions():
    names = []
    for header in (REPO / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_ ]*?\*?\s*\b([a-z][a-z0-9_]*)\s*\(", text, re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(LIB))
    lib.hif8_last_error.restype = ctypes.c_char_p
    return lib


def test_header_declares_the_operator_set():
    names = _declared_functions()
    for required in ("hif8_static_quant", "hif8_scaled_decode", "soft_hif8_gemv", "soft_hif8_gemm",
                     "soft_hif8_static_fused_gemm", "hif8_last_error", "hif8_abi_version"):
        assert required in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.hif8_abi_version() >= 1


def _p(v=1):
    return ctypes.c_void_p(v)


def test_static_quant_rejects_bad_arguments(lib):
    f = lib.hif8_static_quant
    f.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                  ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    assert f(None, 1, 4, 8, _p(), 1, _p(), _p(), None) == 1
    assert b"null pointer" in lib.hif8_last_error()
    assert f(_p(), 1, 3, 8, _p(), 2, _p(), _p(), None) == 1
    assert b"must divide" in lib.hif8_last_error()
    assert f(_p(), 7, 4, 8, _p(), 1, _p(), _p(), None) == 1
    assert b"float16 or bfloat16" in lib.hif8_last_error()


def test_linear_entry_points_enforce_reference_contracts(lib):
    args = [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int] + [ctypes.c_int64] * 3 + [ctypes.c_void_p]
    gemv = lib.soft_hif8_gemv
    gemv.argtypes = args
    assert gemv(_p(), _p(), _p(), _p(), None, -1, _p(), 1, 3, 8, 4, None) == 1
    assert b"M <= 2" in lib.hif8_last_error()
    gemm = lib.soft_hif8_gemm
    gemm.argtypes = args
    assert gemm(_p(), _p(), _p(), _p(), None, -1, _p(), 5, 3, 8, 4, None) == 1
    assert b"output_dtype" in lib.hif8_last_error()
    assert gemm(_p(), _p(), _p(), _p(), None, -1, _p(), 1, 0, 8, 4, None) == 1
    assert b"positive" in lib.hif8_last_error()
    fused = lib.soft_hif8_static_fused_gemm
    fused.argtypes = [ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int] + [ctypes.c_int64] * 3 + [ctypes.c_void_p]
    assert fused(_p(), 1, _p(), _p(), _p(), None, -1, _p(), 1, 5, 8, 4, None) == 1
    assert b"M <= 4" in lib.hif8_last_error()


def test_decoded_weight_entry_points_check_their_contracts(lib):
    """The prefill GEMM over a bf16-decoded weight needs K % 64 == 0, aligned
    operands and a workspace (the decoded activation + split partials, no
    weight copy); the plain decode needs a multiple of 16 elements."""
    size = lib.soft_hif8_gemm_decoded_weight_workspace_size
    size.argtypes = [ctypes.c_int64] * 3
    size.restype = ctypes.c_size_t
    assert size(4096, 24576, 4096) == 4096 * 4096 * 2
    assert size(512, 4096, 4096) == 512 * 4096 * 2 + 4 * 512 * 4096 * 4
    assert size(5, 16, 64) > 0 and size(5, 16, 100) == 0 and size(0, 16, 64) == 0
    f = lib.soft_hif8_gemm_decoded_weight
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int] + \
        [ctypes.c_int64] * 3 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    a16 = _p(256)
    assert f(a16, a16, a16, a16, None, -1, a16, 1, 8, 16, 100, a16, 1 << 20, None) == 2
    assert b"multiple of 64" in lib.hif8_last_error()
    assert f(a16, a16, a16, a16, None, -1, a16, 1, 8, 16, 64, None, 0, None) == 1
    assert b"workspace" in lib.hif8_last_error()
    assert f(a16, _p(258), a16, a16, None, -1, a16, 1, 8, 16, 64, a16, 1 << 20, None) == 1
    assert b"16-byte aligned" in lib.hif8_last_error()
    assert f(a16, None, a16, a16, None, -1, a16, 1, 8, 16, 64, a16, 1 << 20, None) == 1
    assert b"null pointer" in lib.hif8_last_error()
    dec = lib.hif8_decode_bf16
    dec.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    assert dec(a16, a16, 24, None) == 1 and b"multiple of 16" in lib.hif8_last_error()
    assert dec(_p(8), a16, 32, None) == 1 and b"aligned" in lib.hif8_last_error()
    assert dec(a16, a16, 0, None) == 0


def test_gemm_workspace_query_follows_the_split_plan(lib):
    size = lib.soft_hif8_gemm_workspace_size
    size.argtypes = [ctypes.c_int64] * 3
    size.restype = ctypes.c_size_t
    # The workspace is the bf16 copy of A (M*K*2 bytes, rounded to 256), from M = 2048 on
    # also the bf16 copy of W (N*K*2), plus split partials.
    # Enough 256 x 256 tiles to fill the GPU: no split.  GEMV-sized M: no workspace.
    assert size(4096, 24576, 4096) == 4096 * 4096 * 2 + 24576 * 4096 * 2
    # From M = 2048 the plan is the decoded-weight one: k+v at M = 4096 runs
    # 256 unsplit 256 x 128 tiles instead of 128 256-tiles split in two.
    assert size(4096, 2048, 4096) == 4096 * 4096 * 2 + 2048 * 4096 * 2
    assert size(1024, 24576, 4096) == 1024 * 4096 * 2
    assert size(4, 4096, 4096) == 0
    # Prefill M=512 over a 4096 x 4096 projection: 64 tiles of 256 x 128, K split in 4.
    assert size(512, 4096, 4096) == 512 * 4096 * 2 + 4 * 512 * 4096 * 4
    # Splits keep >= 16 K steps of 64 and need N % 4 == 0; K must be a multiple of 64.
    assert size(512, 4096, 1024) == 512 * 1024 * 2
    assert size(512, 4096, 2048) == 512 * 2048 * 2 + 2 * 512 * 4096 * 4
    # Long K: 64 tiles of 256 x 128 split 4 ways (48 steps each) fill the 256 CUs.
    assert size(512, 4096, 12288) == 512 * 12288 * 2 + 4 * 512 * 4096 * 4
    assert size(512, 4094, 4096) == 512 * 4096 * 2
    assert size(300, 16, 100) == 0
    assert size(0, 16, 16) == 0
    ws = lib.soft_hif8_gemm_with_workspace
    ws.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int] + \
        [ctypes.c_int64] * 3 + [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    assert ws(_p(), _p(), _p(), _p(), None, -1, _p(), 1, 512, 4096, 4096, _p(256), 1024, None) == 1
    assert b"workspace" in lib.hif8_last_error()
    assert ws(_p(), _p(), _p(), _p(), None, -1, _p(), 1, 512, 4096, 4096, _p(16), 1 << 30, None) == 1
    assert b"aligned" in lib.hif8_last_error()


def test_prefill_attention_contract_and_workspace_plan(lib):
    """Multi-token paged attention: the workspace follows the plan and invalid
    arguments are rejected before any launch.  Plan: a request whose query
    covers more than two query tiles of 64 rows (rows = tokens x G query heads
    per KV head) is long and takes an image slot - the decoded images of its
    64-key tiles, 66560 bytes each at D=256 - while slots are left: at most
    total_q / (128 / G + 1) of them and as many as fit 512 MiB.  The tile-image
    path runs 128 / G tokens per query tile and splits keys below 256
    workgroups; the in-kernel path runs 64 / G tokens per tile (only the short
    requests' two tiles when every long request has a slot) and splits below
    512 workgroups; two or more 64-key tiles per split; each split partial row
    holds Dv outputs + (max, sum) in fp32."""
    size = lib.hif8_paged_prefill_attention_workspace_size
    size.argtypes = [ctypes.c_int64] * 8
    size.restype = ctypes.c_size_t
    part = (256 + 2) * 4
    # B=1, q 17, ctx 4096, G 4: no long request; 2 query tiles x 4 heads, 64 key tiles in 32 splits of 2.
    assert size(1, 16, 4, 256, 256, 17, 17, 4096) == 1 * 2 * 4 * 32 * 64 * part
    # B=4, q 512: four image slots (4 x 4 heads x 64 tiles); 16 query tiles x 4 heads x 4 fill the
    # 256 workgroups, no split; the in-kernel path keeps 2 query tiles x 4 heads x 4 in 16 splits.
    assert size(4, 16, 4, 256, 256, 2048, 512, 4096) == 4 * 4 * 64 * 66560 + 4 * 2 * 4 * 16 * 64 * part
    # B=1, q 512: one slot + 4 splits of 16 tiles for 16 query tiles x 4 heads of 128 rows.
    assert size(1, 16, 4, 256, 256, 512, 512, 4096) == (4 * 64 * 66560 + 16 * 4 * 4 * 128 * part
                                                         + 1 * 2 * 4 * 32 * 64 * part)
    # Chunked prefill at ctx 16384: one 512-token chunk + 63 decode rows.  At most 575 / 33 = 17
    # requests can be long, 7 slots of 68,157,440 bytes fit 512 MiB; long requests past them run
    # in-kernel, so that path covers all 32 query tiles (8192 items: no split).
    assert size(64, 16, 4, 256, 256, 575, 512, 16384) == 7 * 4 * 256 * 66560
    # Shapes for the one-wavefront kernel need none.
    assert size(1, 12, 4, 64, 64, 17, 17, 4096) == 0 and size(1, 16, 4, 24, 24, 17, 17, 4096) == 0
    assert size(0, 16, 4, 256, 256, 17, 17, 4096) == 0 and size(1, 15, 4, 256, 256, 17, 17, 4096) == 0
    f = lib.hif8_paged_prefill_attention
    f.argtypes = ([ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 5 +
                  [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p] +
                  [ctypes.c_int64] * 5 + [ctypes.c_float, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_size_t, ctypes.c_void_p])
    a = _p(256)

    def call(heads=16, kv_heads=4, d=256, ws=None, ws_bytes=0, query=a, bt_dtype=0, max_seq=4096, q_dtype=1):
        return f(query, q_dtype, a, a, 64, 128, kv_heads, d, d, a, bt_dtype, 32, a, a, 1, heads, 17, 17, max_seq,
                 0.0625, 1, a, ws, ws_bytes, None)

    assert call(heads=15) == 1 and b"divisible by num_kv_heads" in lib.hif8_last_error()
    assert call(d=26) == 1 and b"divisible by four" in lib.hif8_last_error()
    assert call(bt_dtype=5) == 1 and b"int32 or int64" in lib.hif8_last_error()
    assert call(q_dtype=7) == 1 and b"float16 or bfloat16" in lib.hif8_last_error()
    assert call(max_seq=32 * 128 + 1) == 1 and b"block table capacity" in lib.hif8_last_error()
    assert call(query=None) == 1 and b"null pointer" in lib.hif8_last_error()
    assert call() == 1 and b"workspace of" in lib.hif8_last_error()
    assert call(ws=_p(264), ws_bytes=1 << 30) == 1 and b"16-byte aligned" in lib.hif8_last_error()
