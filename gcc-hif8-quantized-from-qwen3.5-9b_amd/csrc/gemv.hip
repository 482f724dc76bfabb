// Decode GEMV (m <= 4) for gfx950: y[m, n] = sum_k dec(a[m,k]) dec(w[n,k]) * ts[m] * cs[n] (+ b[n]).
//
// The weight stream (n*k bytes) dominates and is read exactly once, so the
// kernel is built to keep HBM busy with little VALU work per byte:
//   * a block of 256 threads owns kR consecutive weight rows; thread t owns the
//     16-byte column chunk t (+256 per segment), so each wavefront load covers
//     1 KiB of contiguous row bytes and a thread has kR 16-byte loads in flight;
//   * the activation chunk (m <= 4 rows) is decoded once per chunk into packed
//     bf16 pairs and stays in VGPRs for all kR weight rows;
//   * weight bytes are decoded with a 256-entry bf16 table in LDS (HiF8 is a
//     subset of bf16, so decode is exact) and multiplied with v_dot2_f32_bf16,
//     FP32 accumulation;
//   * partial sums are reduced through LDS (thread-major, padded rows) and the
//     epilogue applies token scale, channel scale and bias, rounding once.
// The fused variant takes fp16/bf16 x and statically encodes it on the fly
// (soft_hif8_fused_gemm.cpp:449-534 with HIF8_FUSED_STATIC_SCALE).
#include "linear.h"

namespace hif8 {
namespace {

constexpr int kThreads = 256;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// 16 HiF8 bytes -> 8 packed bf16 pairs through the LDS decode table.
__device__ __forceinline__ void decode16(const uint16_t *lut, const u32x4 q, uint32_t (&p)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = q[i];
    p[2 * i] = uint32_t(lut[w & 0xFFu]) | (uint32_t(lut[(w >> 8) & 0xFFu]) << 16);
    p[2 * i + 1] = uint32_t(lut[(w >> 16) & 0xFFu]) | (uint32_t(lut[w >> 24]) << 16);
  }
}

// 16 fp16/bf16 values -> static encode with scale s -> decoded bf16 pairs.
template <bool kBf16>
__device__ __forceinline__ void encode_decode16(const uint16_t *x, float s, const uint8_t *enc,
                                                const uint16_t *dec, uint32_t (&p)[8]) {
  const u32x4 a = *reinterpret_cast<const u32x4 *>(x);
  const u32x4 b = *reinterpret_cast<const u32x4 *>(x + 8);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = i < 4 ? a[i] : b[i - 4];
    const float q0 = lo_to_float<kBf16>(w) / s;
    const float q1 = hi_to_float<kBf16>(w) / s;
    const uint32_t c0 = __builtin_isnan(q0) ? uint32_t(kNan) : enc[__float_as_uint(q0) >> 19];
    const uint32_t c1 = __builtin_isnan(q1) ? uint32_t(kNan) : enc[__float_as_uint(q1) >> 19];
    p[i] = uint32_t(dec[c0]) | (uint32_t(dec[c1]) << 16);
  }
}

constexpr int pow2_floor(int v) {
  int p = 1;
  while (p * 2 <= v) p *= 2;
  return p;
}

__device__ __forceinline__ float load_bias(const void *bias, int dtype, int i) {
  const uint16_t h = static_cast<const uint16_t *>(bias)[i];
  return dtype == HIF8_DTYPE_BF16 ? half_bits_to_float<true>(h) : half_bits_to_float<false>(h);
}

__device__ __forceinline__ void store_out(void *out, int dtype, size_t i, float y) {
  static_cast<uint16_t *>(out)[i] =
      dtype == HIF8_DTYPE_BF16 ? float_to_bf16_bits(y) : float_to_f16_bits(y);
}

template <int kM, int kR, int kSrc>
__global__ __launch_bounds__(kThreads, 2) void gemv_kernel(
    const void *__restrict__ act, const float *__restrict__ act_scale,
    const uint8_t *__restrict__ weight, const float *__restrict__ cs,
    const void *__restrict__ bias, int bias_dtype, void *__restrict__ out, int out_dtype,
    int n, int k) {
  constexpr int kV = kR * kM;
  constexpr int kPitch = kV + 4;
  constexpr bool kFused = kSrc != kActCodes;
  __shared__ uint16_t dec_lut[256];
  __shared__ __attribute__((aligned(16))) uint8_t enc_lut[kFused ? 8192 : 16];
  __shared__ __attribute__((aligned(16))) float red[kThreads * kPitch];

  const int tid = threadIdx.x;
  dec_lut[tid] = kDeviceTables.decode_bf16[tid];
  if constexpr (kFused) {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(kDeviceTables.static_encode);
    u32x4 *dst = reinterpret_cast<u32x4 *>(enc_lut);
    dst[tid] = src[tid];
    dst[tid + kThreads] = src[tid + kThreads];
  }
  __syncthreads();

  const int n0 = blockIdx.x * kR;
  const int chunks = k >> 4;
  const float fixed = kFused ? act_scale[0] : 0.f;
  float acc[kR][kM];
#pragma unroll
  for (int r = 0; r < kR; ++r)
#pragma unroll
    for (int m = 0; m < kM; ++m) acc[r][m] = 0.f;

  for (int c = tid; c < chunks; c += kThreads) {
    u32x4 wq[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      // Rows past n re-read row n-1; their sums are never stored.
      const int row = min(n0 + r, n - 1);
      wq[r] = reinterpret_cast<const u32x4 *>(weight + size_t(row) * k)[c];
    }
    uint32_t a[kM][8];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      if constexpr (kFused) {
        encode_decode16<kSrc == kActBf16>(static_cast<const uint16_t *>(act) + size_t(m) * k + 16 * c,
                                          fixed, enc_lut, dec_lut, a[m]);
      } else {
        decode16(dec_lut, reinterpret_cast<const u32x4 *>(static_cast<const uint8_t *>(act) + size_t(m) * k)[c], a[m]);
      }
    }
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      uint32_t p[8];
      decode16(dec_lut, wq[r], p);
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int m = 0; m < kM; ++m) acc[r][m] = dot2(a[m][j], p[j], acc[r][m]);
    }
  }

  // Thread-major partials, then column sums by kTpo threads per output.
  float *mine = red + tid * kPitch;
#pragma unroll
  for (int v = 0; v < kV; v += 4) {
    float4 f;
    f.x = acc[(v + 0) / kM][(v + 0) % kM];
    f.y = acc[(v + 1) / kM][(v + 1) % kM];
    f.z = acc[(v + 2) / kM][(v + 2) % kM];
    f.w = acc[(v + 3) / kM][(v + 3) % kM];
    *reinterpret_cast<float4 *>(mine + v) = f;
  }
  __syncthreads();
  constexpr int kTpo = pow2_floor(kThreads / kV) > 64 ? 64 : pow2_floor(kThreads / kV);
  const int v = tid / kTpo;
  const int part = tid % kTpo;
  float s = 0.f;
  if (v < kV) {
#pragma unroll 4
    for (int t = part; t < kThreads; t += kTpo) s += red[t * kPitch + v];
  }
#pragma unroll
  for (int off = kTpo / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
  if (v < kV && part == 0) {
    const int r = v / kM, m = v % kM;
    const int row = n0 + r;
    if (row < n) {
      const float ts = kFused ? fixed : act_scale[m];
      float y = s * ts * cs[row];
      if (bias) y += load_bias(bias, bias_dtype, row);
      store_out(out, out_dtype, size_t(m) * n + row, y);
    }
  }
}

// Any shape or alignment: one wavefront per output row, byte-wise k loop.
__global__ __launch_bounds__(64) void gemv_simple_kernel(
    const void *__restrict__ act, int act_kind, const float *__restrict__ act_scale,
    const uint8_t *__restrict__ weight, const float *__restrict__ cs,
    const void *__restrict__ bias, int bias_dtype, void *__restrict__ out, int out_dtype,
    int m_rows, int n, int k) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const float fixed = act_kind == kActCodes ? 0.f : act_scale[0];
  for (int kk = lane; kk < k; kk += kWave) {
    const float wv = __uint_as_float(kDeviceTables.decode_f32[weight[size_t(row) * k + kk]]);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m < m_rows) {
        uint32_t code;
        if (act_kind == kActCodes) {
          code = static_cast<const uint8_t *>(act)[size_t(m) * k + kk];
        } else {
          const uint16_t h = static_cast<const uint16_t *>(act)[size_t(m) * k + kk];
          const float xv = act_kind == kActBf16 ? half_bits_to_float<true>(h) : half_bits_to_float<false>(h);
          code = static_encode_bits(__float_as_uint(xv / fixed));
        }
        acc[m] = fmaf(__uint_as_float(kDeviceTables.decode_f32[code]), wv, acc[m]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) acc[m] = wave_sum(acc[m]);
  if (lane < m_rows) {
    const int m = lane;
    const float a = m == 0 ? acc[0] : (m == 1 ? acc[1] : (m == 2 ? acc[2] : acc[3]));
    const float ts = act_kind == kActCodes ? act_scale[m] : fixed;
    float y = a * ts * cs[row];
    if (bias) y += load_bias(bias, bias_dtype, row);
    store_out(out, out_dtype, size_t(m) * n + row, y);
  }
}

template <int kM, int kR>
void dispatch_src(const LinearArgs &a, dim3 grid) {
  const int n = int(a.n), k = int(a.k);
  switch (a.act_kind) {
    case kActCodes:
      gemv_kernel<kM, kR, kActCodes><<<grid, kThreads, 0, a.stream>>>(
          a.act, a.act_scale, a.weight, a.channel_scale, a.bias, a.bias_dtype, a.out, a.out_dtype, n, k);
      break;
    case kActF16:
      gemv_kernel<kM, kR, kActF16><<<grid, kThreads, 0, a.stream>>>(
          a.act, a.act_scale, a.weight, a.channel_scale, a.bias, a.bias_dtype, a.out, a.out_dtype, n, k);
      break;
    default:
      gemv_kernel<kM, kR, kActBf16><<<grid, kThreads, 0, a.stream>>>(
          a.act, a.act_scale, a.weight, a.channel_scale, a.bias, a.bias_dtype, a.out, a.out_dtype, n, k);
      break;
  }
}

template <int kR>
void dispatch_m(const LinearArgs &a) {
  const dim3 grid(unsigned((a.n + kR - 1) / kR));
  switch (a.m) {
    case 1: dispatch_src<1, kR>(a, grid); break;
    case 2: dispatch_src<2, kR>(a, grid); break;
    case 3: dispatch_src<3, kR>(a, grid); break;
    default: dispatch_src<4, kR>(a, grid); break;
  }
}

}  // namespace

int launch_gemv(const LinearArgs &a) {
  if (a.m < 1 || a.m > 4) return fail(HIF8_ERR_UNSUPPORTED, "GEMV kernel handles 1 <= M <= 4, got %lld", (long long)a.m);
  const bool vec = a.k % 16 == 0 && aligned(a.weight, 16) && aligned(a.act, 16);
  if (!vec) {
    gemv_simple_kernel<<<dim3(unsigned(a.n)), 64, 0, a.stream>>>(
        a.act, a.act_kind, a.act_scale, a.weight, a.channel_scale, a.bias, a.bias_dtype, a.out,
        a.out_dtype, int(a.m), int(a.n), int(a.k));
  } else if (a.n >= 16384) {
    dispatch_m<16>(a);
  } else if (a.n >= 4096) {
    dispatch_m<8>(a);
  } else {
    dispatch_m<4>(a);
  }
  return check_launch("soft_hif8 GEMV");
}

}  // namespace hif8
