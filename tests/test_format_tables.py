"""The device tables are built by constexpr code in csrc/hif8_format.h.  The
header is plain C++ on the host, so compile it with g++ and compare every entry
with the (golden-pinned) oracle tables, plus the arithmetic static encoder on
every bf16 input scaled by a few divisors (CPU only)."""

import ctypes
import subprocess

import numpy as np
import pytest

from conftest import PKG_ROOT
from oracle import hif8_oracle as o

SRC = r"""
#include <stdint.h>
#include <string.h>
#include "hif8_format.h"
static constexpr hif8::Tables kT = hif8::make_tables();
extern "C" void dump_tables(uint8_t *enc, uint16_t *bf16, uint32_t *f32, uint16_t *f16) {
  memcpy(enc, kT.static_encode, sizeof(kT.static_encode));
  memcpy(f16, kT.decode_f16, sizeof(kT.decode_f16));
  memcpy(bf16, kT.decode_bf16, sizeof(kT.decode_bf16));
  memcpy(f32, kT.decode_f32, sizeof(kT.decode_f32));
}
extern "C" void static_encode_f32(const uint32_t *bits, uint8_t *out, long n) {
  for (long i = 0; i < n; ++i) out[i] = (uint8_t)hif8::static_encode_bits(bits[i]);
}
"""


@pytest.fixture(scope="module")
def fmt(tmp_path_factory):
    d = tmp_path_factory.mktemp("fmt")
    (d / "fmt.cpp").write_text(SRC)
    so = d / "libfmt.so"
    subprocess.run(["g++", "-std=c++17", "-O1", "-fconstexpr-ops-limit=1000000000", "-shared", "-fPIC",
                    f"-I{PKG_ROOT / 'csrc'}", str(d / "fmt.cpp"), "-o", str(so)], check=True)
    lib = ctypes.CDLL(str(so))
    lib.dump_tables.argtypes = [ctypes.c_void_p] * 4
    lib.static_encode_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long]
    return lib


def test_constexpr_tables_equal_oracle(fmt):
    enc = np.zeros(8192, np.uint8)
    bf = np.zeros(256, np.uint16)
    f32 = np.zeros(256, np.uint32)
    f16 = np.zeros(256, np.uint16)
    fmt.dump_tables(enc.ctypes.data, bf.ctypes.data, f32.ctypes.data, f16.ctypes.data)
    assert np.array_equal(enc, o.STATIC_LUT)
    want_bf = np.array([o.bf16_bits_of_decode(b) for b in range(256)], np.uint16)
    assert np.array_equal(bf, want_bf)
    want_f32 = o.DECODE_F32.view(np.uint32).copy()
    want_f32[o.NAN_CODE] = 0x7FC00000
    assert np.array_equal(f32, want_f32)
    want_f16 = np.array([o.half_bits_of_decode(b) for b in range(256)], np.uint16)
    assert np.array_equal(f16, want_f16)
    # Exactness: the fp16 payload converts back to the fp32 value.
    finite = np.isfinite(o.DECODE_F32)
    assert np.array_equal(f16.view(np.float16).astype(np.float32)[finite], o.DECODE_F32[finite])


def test_arithmetic_static_encoder_on_all_bf16_quotients(fmt):
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    for s in (1.0, 0.75, 2.0 ** -10, 3.0e-5, 1234.5, 2.0 ** 100):
        with np.errstate(all="ignore"):
            q = (x / np.float32(s)).astype(np.float32)
        got = np.zeros(q.size, np.uint8)
        fmt.static_encode_f32(q.view(np.uint32).ctypes.data, got.ctypes.data, q.size)
        assert np.array_equal(got, o.saturating_encode_array(q)), s


def test_arithmetic_static_encoder_on_random_fp32(fmt):
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2 ** 32, 1_000_000, dtype=np.uint64).astype(np.uint32)
    got = np.zeros(bits.size, np.uint8)
    fmt.static_encode_f32(bits.ctypes.data, got.ctypes.data, bits.size)
    assert np.array_equal(got, o.saturating_encode_array(bits.view(np.float32)))
