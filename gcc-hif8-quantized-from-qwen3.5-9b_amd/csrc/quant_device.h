// Device-side static HiF8 encode of 16 fp16/bf16 values, shared by the
// standalone static quant and the fused KV-cache write.
//
// Contract (calibration.py:182-201; hif8_static_quant.cpp:67-89):
//   q = float(x) / s   (IEEE round-to-nearest division)
//   byte = static_encode(q)   (finite clamped to +-2^15, ties away, no -0)
//
// The encoder multiplies by a per-row reciprocal instead of dividing.  The
// product x * rcp(s) is within 1.5 ulp (relative) of x/s and the correctly
// rounded quotient within 0.5 ulp, so the two fp32 bit patterns differ by at
// most 3.  The encode depends only on bits 31..19 (the 13-bit index of the
// static table), so only a product within a few ulps of a multiple of 2^19,
// or a NaN, can encode differently; such elements are redone with a true IEEE
// division (margin 8 ulps).  The encode itself is one lookup in the 8 KiB
// static table, staged in LDS by the caller.
#pragma once

#include "hif8_common.h"

namespace hif8 {

constexpr uint32_t kNearMargin = 8;

__device__ __forceinline__ bool near_index_boundary(float q) {
  const uint32_t u = __float_as_uint(q);
  return (((u + kNearMargin) & 0x7FFFFu) <= 2u * kNearMargin) || __builtin_isnan(q);
}

// Copies the 8 KiB static encode table into LDS; the caller synchronises.
__device__ __forceinline__ void stage_static_encode_table(uint8_t *lut, int tid, int nthreads) {
  const uint4 *src = reinterpret_cast<const uint4 *>(kDeviceTables.static_encode);
  uint4 *dst = reinterpret_cast<uint4 *>(lut);
  for (int i = tid; i < 8192 / 16; i += nthreads) dst[i] = src[i];
}

// 16 consecutive fp16/bf16 values from a 16-byte aligned address.
template <bool kBf16>
__device__ __forceinline__ void load16(const uint16_t *p, float (&v)[16]) {
  const uint4 a = *reinterpret_cast<const uint4 *>(p);
  const uint4 b = *reinterpret_cast<const uint4 *>(p + 8);
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[2 * i] = lo_to_float<kBf16>(w[i]);
    v[2 * i + 1] = hi_to_float<kBf16>(w[i]);
  }
}

__device__ __forceinline__ uint32_t encode_q(float q, const uint8_t *lut) {
  return lut[__float_as_uint(q) >> 19];
}

// Encodes xf[j] / s (j = 0..15) into four little-endian words of codes.
__device__ __forceinline__ void static_encode16(const float (&xf)[16], float s, const uint8_t *lut,
                                                uint32_t (&w)[4]) {
  const float r = __builtin_amdgcn_rcpf(s);
  float q[16];
  // One decision for the 16 products: the smallest distance to an index
  // boundary (a min tree) and whether any product of the wavefront is NaN
  // (pairwise unordered compares into a lane mask; a NaN anywhere sends the
  // whole wavefront down the exact path, which encodes every value alike).
  uint32_t nearest = 0xFFFFFFFFu;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    q[j] = xf[j] * r;
    // Bits 18..0 of u + margin, moved to the top (one add-shift).
    nearest = min(nearest, (__float_as_uint(q[j]) + kNearMargin) << 13);
  }
  uint64_t nan_lanes = 0;
#pragma unroll
  for (int j = 0; j < 16; j += 2) nan_lanes |= __builtin_amdgcn_fcmpf(q[j], q[j + 1], 8);  // FCMP_UNO
  const bool redo = nearest <= (2u * kNearMargin) << 13 || nan_lanes != 0;
  if (__builtin_expect(!redo, 1)) {
    // No value is NaN or near an index boundary: the product encodes exactly
    // like the correctly rounded quotient.  Bytes 0 and 2 (1 and 3) of a
    // word are looked up into the two halves of one register, then merged.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
      u16x2_t even, odd;
      even.x = lut[__float_as_uint(q[4 * i]) >> 19];
      even.y = lut[__float_as_uint(q[4 * i + 2]) >> 19];
      odd.x = lut[__float_as_uint(q[4 * i + 1]) >> 19];
      odd.y = lut[__float_as_uint(q[4 * i + 3]) >> 19];
      w[i] = __builtin_bit_cast(uint32_t, even) | (__builtin_bit_cast(uint32_t, odd) << 8);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // NaN is decided by the full mantissa, as the reference codec does.
        const float v = xf[4 * i + j] / s;
        b[j] = __builtin_isnan(v) ? uint32_t(kNan) : encode_q(v, lut);
      }
      w[i] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    }
  }
}

}  // namespace hif8
