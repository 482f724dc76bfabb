// hif8_static_quant and hif8_scaled_decode for gfx950.
//
// Static quant contract (calibration.py:182-201; hif8_static_quant.cpp:67-89):
//   q = float(x) / scale[r % S]   (IEEE round-to-nearest division)
//   byte = static_encode(q)       (finite clamped to +-2^15, ties away, no -0)
//
// The vector kernel is HBM-bound (2 B in + 1 B out per element), so it spends
// as few VALU cycles per element as possible: static_encode16 multiplies by a
// per-row reciprocal and falls back to an IEEE division only next to an
// encode-index boundary (the argument is spelled out in quant_device.h).
#include <stdlib.h>

#include <algorithm>

#include "quant_device.h"

namespace hif8 {
namespace {

constexpr int kThreads = 256;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// The vector kernel always stages the 8 KiB table: measured on MI355X, the
// table-free arithmetic encoder is ~3x slower even for a single block
// (M=1, K=4096: 10.2 vs 3.4 us) because of its data-dependent branches.

// One thread = 16 consecutive elements of one row (requires k % 16 == 0 and
// 16-byte aligned x / data); grid-stride over the chunks with the next chunk
// loaded while the current one is encoded.  The 8 KiB table is staged once
// per workgroup (grids of up to 32 per CU, at most a few chunks per thread:
// more workgroups measured faster than fewer walking more chunks, M=4096
// K=12288 32.2 -> 29.8 us against 16 per CU): its loads go first, then the first
// chunk's, so the table's LDS stores wait only for the table (loads return in
// order) and the barrier, which waits for LDS traffic only, leaves the chunk
// in flight.  One encode in the loop body keeps the kernel small: a launch
// this short pays for every instruction it fetches cold.
// kRowScales: more than one fixed scale (row r uses fixed[r % scale_count]);
// with one, no chunk needs its row index and the loop has no division.  The
// per-row output scales are written before the loop, one row per thread.
template <bool kBf16, bool kRowScales>
__global__ __launch_bounds__(kThreads) void static_quant_vec16(
    const uint16_t *__restrict__ x, const float *__restrict__ fixed, uint8_t *__restrict__ out,
    float *__restrict__ row_scale, uint32_t n_chunks, uint32_t k_chunks, uint32_t scale_count, uint32_t rows) {
  __shared__ __attribute__((aligned(16))) uint8_t lut[8192];
  static_assert(8192 == 2 * 16 * kThreads, "two 16-byte table words per thread");
  const uint4 *tsrc = reinterpret_cast<const uint4 *>(kDeviceTables.static_encode);
  const uint4 t0 = tsrc[threadIdx.x], t1 = tsrc[threadIdx.x + kThreads];
  const uint64_t stride = uint64_t(gridDim.x) * kThreads;
  uint64_t c = uint64_t(blockIdx.x) * kThreads + threadIdx.x;  // 64-bit: no wrap near 2^32 chunks
  // A chunk's data (and with kRowScales its row's scale) are loaded
  // together, one chunk ahead.
  uint4 a0{}, a1{};
  float sc = kRowScales ? 0.f : fixed[0];
  // Unconditional loads (a chunk past the end reloads the last one, unused),
  // so the compiler can count them and wait for exactly the ones it needs.
  auto fetch = [&](uint64_t ch) {
    const uint64_t safe = ch < n_chunks ? ch : n_chunks - 1;
    const uint4 *src = reinterpret_cast<const uint4 *>(x + safe * 16);
    a0 = src[0];
    a1 = src[1];
    if constexpr (kRowScales) sc = fixed[(uint32_t(safe) / k_chunks) % scale_count];
  };
  fetch(c);
  for (uint64_t r = c; r < rows; r += stride) row_scale[r] = fixed[kRowScales ? uint32_t(r) % scale_count : 0u];
  reinterpret_cast<uint4 *>(lut)[threadIdx.x] = t0;
  reinterpret_cast<uint4 *>(lut)[threadIdx.x + kThreads] = t1;
  lds_barrier();
  for (; c < n_chunks; c += stride) {
    const uint32_t v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float s = sc;
    fetch(c + stride);
    float xf[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xf[2 * i] = lo_to_float<kBf16>(v[i]);
      xf[2 * i + 1] = hi_to_float<kBf16>(v[i]);
    }
    uint32_t w[4];
    static_encode16(xf, s, lut, w);
    // Non-temporal store (M=4096, K=4096: 13.35 -> 12.33 us on MI355X; the
    // same hint on the loads measured slower).
    __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4 *>(out + c * 16));
  }
}

// Any shape / alignment: one thread per element, true division, arithmetic encode.
template <bool kBf16>
__global__ __launch_bounds__(kThreads) void static_quant_scalar(
    const uint16_t *__restrict__ x, const float *__restrict__ fixed, uint8_t *__restrict__ out,
    float *__restrict__ row_scale, uint64_t n, uint64_t k, uint32_t scale_count) {
  const uint64_t stride = uint64_t(gridDim.x) * kThreads;
  for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
    const uint64_t row = i / k;
    const float s = fixed[row % scale_count];
    if (i == row * k) row_scale[row] = s;
    const float q = half_bits_to_float<kBf16>(x[i]) / s;
    out[i] = uint8_t(static_encode_bits(__float_as_uint(q)));
  }
}

// ------------------------------------------------------------ scaled decode

template <bool kVec>
__global__ __launch_bounds__(kThreads) void scaled_decode_kernel(
    const uint8_t *__restrict__ data, const float *__restrict__ scale, uint16_t *__restrict__ out,
    uint64_t rows, uint64_t k, uint64_t stride_bytes) {
  __shared__ uint32_t lut[256];
  for (int i = threadIdx.x; i < 256; i += kThreads) lut[i] = kDeviceTables.decode_f32[i];
  __syncthreads();
  const uint64_t per_row = kVec ? k / 16 : k;
  const uint64_t total = rows * per_row;
  const uint64_t step = uint64_t(gridDim.x) * kThreads;
  for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < total; i += step) {
    const uint64_t row = i / per_row;
    const uint64_t col = (i - row * per_row) * (kVec ? 16 : 1);
    const float s = scale[row];
    const uint8_t *src = data + row * stride_bytes + col;
    uint16_t *dst = out + row * k + col;
    if constexpr (kVec) {
      const uint4 q = *reinterpret_cast<const uint4 *>(src);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
      uint32_t o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t word = w[j >> 1] >> ((j & 1) * 16);
        const float v0 = __uint_as_float(lut[word & 0xFFu]) * s;
        const float v1 = __uint_as_float(lut[(word >> 8) & 0xFFu]) * s;
        const uint32_t h0 = __builtin_isnan(v0) ? kBf16Nan : float_to_bf16_bits(v0);
        const uint32_t h1 = __builtin_isnan(v1) ? kBf16Nan : float_to_bf16_bits(v1);
        o[j] = h0 | (h1 << 16);
      }
      uint4 *d = reinterpret_cast<uint4 *>(dst);
      d[0] = make_uint4(o[0], o[1], o[2], o[3]);
      d[1] = make_uint4(o[4], o[5], o[6], o[7]);
    } else {
      const float v = __uint_as_float(lut[*src]) * s;
      *dst = __builtin_isnan(v) ? kBf16Nan : float_to_bf16_bits(v);
    }
  }
}

// Dynamic per-row quantisation (the legacy W8A8HIF8_SOFT activations;
// hif8_dynamic_quant.cpp:35-200):
//   scale[r] = max(max |x[r, :]| over the finite values, 1e-12)
//   q = x * RN(1 / scale)   when k % 32 == 0 (the reference's vector path),
//       x / scale           otherwise (its scalar path)
//   data = encode(q): NaN -> 0x80, Inf kept, zero magnitude unsigned.
// |q| <= 1 + 1 ulp for finite x, far below the static table's saturation
// point (1.25 * 2^15), so the static table gives the plain signed encode.
// One block per row (grid-stride), 16 elements per thread and pass when
// k % 16 == 0 and the row is 16-byte aligned.
template <bool kBf16, bool kVec>
__global__ __launch_bounds__(kThreads) void dynamic_quant_kernel(const uint16_t *__restrict__ x,
                                                                 uint8_t *__restrict__ out,
                                                                 float *__restrict__ row_scale, uint32_t rows,
                                                                 uint32_t k) {
  __shared__ __attribute__((aligned(16))) uint8_t lut[8192];
  __shared__ float red[kThreads / kWave];
  stage_static_encode_table(lut, threadIdx.x, kThreads);
  __syncthreads();
  const bool by_reciprocal = k % 32 == 0;
  const uint32_t chunks = kVec ? k / 16 : k;
  for (uint32_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const uint16_t *xr = x + size_t(row) * k;
    float m = 0.f;
    for (uint32_t c = threadIdx.x; c < chunks; c += kThreads) {
      if constexpr (kVec) {
        float v[16];
        load16<kBf16>(xr + size_t(c) * 16, v);
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (__builtin_isfinite(v[j])) m = fmaxf(m, fabsf(v[j]));
      } else {
        const float v = half_bits_to_float<kBf16>(xr[c]);
        if (__builtin_isfinite(v)) m = fmaxf(m, fabsf(v));
      }
    }
    m = wave_max(m);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = m;
    __syncthreads();
    float amax = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / kWave; ++w) amax = fmaxf(amax, red[w]);
    const float s = fmaxf(amax, 1.0e-12f);
    const float r = 1.0f / s;  // IEEE division (built with correctly rounded division)
    auto encode = [&](float v) -> uint32_t {
      const float q = by_reciprocal ? v * r : v / s;
      return __builtin_isnan(q) ? uint32_t(kNan) : uint32_t(lut[__float_as_uint(q) >> 19]);
    };
    uint8_t *orow = out + size_t(row) * k;
    for (uint32_t c = threadIdx.x; c < chunks; c += kThreads) {
      if constexpr (kVec) {
        float v[16];
        load16<kBf16>(xr + size_t(c) * 16, v);
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[i] = encode(v[4 * i]) | (encode(v[4 * i + 1]) << 8) | (encode(v[4 * i + 2]) << 16) |
                 (encode(v[4 * i + 3]) << 24);
        *reinterpret_cast<uint4 *>(orow + size_t(c) * 16) = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
        orow[c] = uint8_t(encode(half_bits_to_float<kBf16>(xr[c])));
      }
    }
    if (threadIdx.x == 0) row_scale[row] = s;
    __syncthreads();  // red is reused by the next row
  }
}

int grid_for(uint64_t work_items, int per_cu) {
  uint64_t blocks = (work_items + kThreads - 1) / kThreads;
  const uint64_t cap = uint64_t(256) * per_cu;  // 256 CUs on MI355X
  if (blocks > cap) blocks = cap;
  return int(blocks < 1 ? 1 : blocks);
}

}  // namespace
}  // namespace hif8

using namespace hif8;

extern "C" int hif8_static_quant(const void *x, int x_dtype, int64_t rows, int64_t k,
                                 const float *fixed_scale, int64_t scale_count, uint8_t *data,
                                 float *row_scale, hif8_stream_t stream) {
  clear_error();
  if (!x || !fixed_scale || !data || !row_scale)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_static_quant: null pointer argument");
  if (!is_io_dtype(x_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_static_quant: x must be float16 or bfloat16");
  if (rows <= 0 || k <= 0 || scale_count <= 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_static_quant: dimensions must be positive");
  if (rows % scale_count)
    return fail(HIF8_ERR_INVALID_ARGUMENT,
                "hif8_static_quant: fixed_scale count must divide the activation row count");
  if (rows > 0xFFFFFFFFll || k > 0xFFFFFFFFll || scale_count > 0xFFFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_static_quant: dimensions must fit uint32");
  const bool bf16 = x_dtype == HIF8_DTYPE_BF16;
  const uint64_t n = uint64_t(rows) * uint64_t(k);
  const uint64_t n_chunks = n / 16;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint16_t *xs = static_cast<const uint16_t *>(x);
  if (k % 16 == 0 && aligned(x, 16) && aligned(data, 16) && n_chunks <= 0xFFFFFFFFull) {
    const dim3 grid(grid_for(n_chunks, 32)), block(kThreads);
    const uint32_t nc = uint32_t(n_chunks), kc = uint32_t(k / 16), sc = uint32_t(scale_count), r = uint32_t(rows);
    if (sc == 1) {
      if (bf16) static_quant_vec16<true, false><<<grid, block, 0, s>>>(xs, fixed_scale, data, row_scale, nc, kc, sc, r);
      else static_quant_vec16<false, false><<<grid, block, 0, s>>>(xs, fixed_scale, data, row_scale, nc, kc, sc, r);
    } else {
      if (bf16) static_quant_vec16<true, true><<<grid, block, 0, s>>>(xs, fixed_scale, data, row_scale, nc, kc, sc, r);
      else static_quant_vec16<false, true><<<grid, block, 0, s>>>(xs, fixed_scale, data, row_scale, nc, kc, sc, r);
    }
  } else {
    const dim3 grid(grid_for(n, 8)), block(kThreads);
    if (bf16) static_quant_scalar<true><<<grid, block, 0, s>>>(xs, fixed_scale, data, row_scale, n, uint64_t(k), uint32_t(scale_count));
    else static_quant_scalar<false><<<grid, block, 0, s>>>(xs, fixed_scale, data, row_scale, n, uint64_t(k), uint32_t(scale_count));
  }
  return check_launch("hif8_static_quant");
}

extern "C" int hif8_dynamic_quant(const void *x, int x_dtype, int64_t rows, int64_t k, uint8_t *data,
                                  float *row_scale, hif8_stream_t stream) {
  clear_error();
  if (!x || !data || !row_scale) return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_dynamic_quant: null pointer argument");
  if (!is_io_dtype(x_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_dynamic_quant: x must be float16 or bfloat16");
  if (rows <= 0 || k <= 0) return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_dynamic_quant: dimensions must be positive");
  if (rows > 0xFFFFFFFFll || k > 0xFFFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_dynamic_quant: dimensions must fit uint32");
  const bool bf16 = x_dtype == HIF8_DTYPE_BF16;
  const bool vec = k % 16 == 0 && aligned(x, 16) && aligned(data, 16);
  const dim3 grid(unsigned(std::min<int64_t>(rows, 2048))), block(kThreads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const uint16_t *xs = static_cast<const uint16_t *>(x);
  const uint32_t r = uint32_t(rows), kk = uint32_t(k);
  if (bf16) {
    if (vec) dynamic_quant_kernel<true, true><<<grid, block, 0, s>>>(xs, data, row_scale, r, kk);
    else dynamic_quant_kernel<true, false><<<grid, block, 0, s>>>(xs, data, row_scale, r, kk);
  } else {
    if (vec) dynamic_quant_kernel<false, true><<<grid, block, 0, s>>>(xs, data, row_scale, r, kk);
    else dynamic_quant_kernel<false, false><<<grid, block, 0, s>>>(xs, data, row_scale, r, kk);
  }
  return check_launch("hif8_dynamic_quant");
}

extern "C" int hif8_scaled_decode(const uint8_t *data, int64_t rows, int64_t k,
                                  int64_t data_row_stride, const float *scale, uint16_t *out,
                                  hif8_stream_t stream) {
  clear_error();
  if (!data || !scale || !out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_scaled_decode: null pointer argument");
  if (rows <= 0 || k <= 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_scaled_decode: dimensions must be positive");
  if (data_row_stride < k)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_scaled_decode: row stride %lld < k %lld",
                (long long)data_row_stride, (long long)k);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = k % 16 == 0 && data_row_stride % 16 == 0 && aligned(data, 16) && aligned(out, 16);
  const uint64_t items = uint64_t(rows) * uint64_t(vec ? k / 16 : k);
  const dim3 grid(grid_for(items, 8)), block(kThreads);
  if (vec) scaled_decode_kernel<true><<<grid, block, 0, s>>>(data, scale, out, rows, k, data_row_stride);
  else scaled_decode_kernel<false><<<grid, block, 0, s>>>(data, scale, out, rows, k, data_row_stride);
  return check_launch("hif8_scaled_decode");
}
