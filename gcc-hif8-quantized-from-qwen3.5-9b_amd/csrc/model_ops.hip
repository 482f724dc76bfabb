// Decode-step glue of the synthetic hybrid model (the config-5 workload),
// fused so that one decode step is a few launches per layer instead of tens
// of elementwise ones.  None of these is a HiF8 operator; they are the bf16 /
// fp32 parts the reference leaves to the model (norms, the MLP activation,
// the linear-attention conv and recurrence).
//
//   hif8_add_rms_norm     h <- bf16(h + delta) (optional), out = bf16(h * rsqrt(mean(h^2) + eps) * w)
//   hif8_silu_mul         out[r, i] = bf16(silu(gu[r, i]) * gu[r, n + i])
//   hif8_gdn_decode_step  one token of the gated delta rule per request and value head:
//       causal depthwise conv over the q|k|v channels with the carried state, SiLU;
//       q, k L2-normalised (q also / sqrt(dk)), k/q heads shared by v_heads / k_heads
//       value heads; beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias);
//       S <- e^g S;  S <- S + k (beta (v - S^T k))^T;  o = S^T q;
//       out = bf16(rms_norm(o) * w_out * silu(z)).
//   hif8_bf16_gemv        out = bf16(x w^T) for M <= 4 (the small bf16 projections)
//   hif8_qk_norm_rope     per-head RMSNorm of q and k, rotary embedding on the
//       first rotary_dim dims (neox halves), v split off, cache slots.
#include <math.h>

#include <algorithm>

#include "hif8_common.h"
#include "hif8_rocm.h"
#include "quant_device.h"

namespace hif8 {
namespace {

__device__ __forceinline__ float bf(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }
__device__ __forceinline__ uint16_t to_bf(float f) { return float_to_bf16_bits(f); }

template <int kThreads>
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave;
  __syncthreads();  // red may still be read by a previous reduction
  if (threadIdx.x % kWave == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / kWave; ++i) s += red[i];
  return s;
}

constexpr int kNormThreads = 256;

template <bool kResidual>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(uint16_t *__restrict__ h,
                                                                    const uint16_t *__restrict__ delta,
                                                                    const uint16_t *__restrict__ w,
                                                                    uint16_t *__restrict__ out, int n, float eps) {
  __shared__ float red[kNormThreads / kWave];
  uint16_t *hr = h + size_t(blockIdx.x) * n;
  const uint16_t *dr = kResidual ? delta + size_t(blockIdx.x) * n : nullptr;
  uint16_t *orow = out + size_t(blockIdx.x) * n;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += kNormThreads) {
    float v = bf(hr[i]);
    if constexpr (kResidual) {
      const uint16_t s = to_bf(v + bf(dr[i]));  // the residual stream is bf16
      hr[i] = s;
      v = bf(s);
    }
    ss += v * v;
  }
  const float r = rsqrtf(block_sum<kNormThreads>(ss, red) / float(n) + eps);
  for (int i = threadIdx.x; i < n; i += kNormThreads) orow[i] = to_bf(bf(hr[i]) * r * bf(w[i]));
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ gu, uint16_t *__restrict__ out,
                                                       int64_t rows, int n) {
  const int64_t total = rows * n;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / n, c = i - r * n;
    const float g = bf(gu[r * 2 * n + c]), u = bf(gu[r * 2 * n + n + c]);
    out[i] = to_bf(g / (1.f + expf(-g)) * u);
  }
}

// Conv over channel c of request b: out = silu(sum_j w[c, j] seq[j]),
// seq = (state[b, c, 0 .. K-2], x); the state shifts by one.
__global__ __launch_bounds__(256) void gdn_conv_kernel(const uint16_t *__restrict__ mixed, int64_t ld, int channels,
                                                       const uint16_t *__restrict__ w, uint16_t *__restrict__ state,
                                                       float *__restrict__ out, int batch, int kw) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= batch * channels) return;
  const int b = idx / channels, c = idx - b * channels;
  uint16_t *st = state + size_t(idx) * (kw - 1);
  const uint16_t x = mixed[size_t(b) * ld + c];
  float acc = 0.f;
  for (int j = 0; j < kw - 1; ++j) acc += bf(st[j]) * bf(w[size_t(c) * kw + j]);
  acc += bf(x) * bf(w[size_t(c) * kw + kw - 1]);
  for (int j = 0; j + 1 < kw - 1; ++j) st[j] = st[j + 1];
  st[kw - 2] = x;
  out[idx] = acc / (1.f + expf(-acc));
}

// Rows of n % 8 == 0, n <= 8 * kRowThreads * kRowChunks, 16-byte aligned:
// thread t owns 16-byte chunks t + kRowThreads * c, loads all of them at
// once and keeps the row in registers (the scalar loop above waits on one
// 2-byte load per iteration and re-reads the row: ~10 us for n = 4096).  A
// decode row runs on one block, so its latency is the block's: 512 threads
// (one chunk each at n = 4096) take 3.2 us per add + norm + quant on MI355X
// where 256 threads take 4.3 us and 1024 threads 3.4 us.
constexpr int kRowThreads = 512, kRowChunks = 2;

// Static HiF8 codes of eight bf16 values (four packed pairs) divided by s,
// as hif8_static_quant encodes them: the product with the reciprocal, or the
// IEEE quotient for an element near an encode-index boundary or NaN.  Both
// encode alike everywhere else, so the per-element choice gives the codes of
// the standalone quant whatever its grouping.
__device__ __forceinline__ uint2 static_encode8(const uint32_t (&pairs)[4], float s, const uint8_t *lut) {
  const float r = __builtin_amdgcn_rcpf(s);
  uint32_t b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w = pairs[j / 2];
    const float x = __uint_as_float(j % 2 ? (w & 0xFFFF0000u) : (w << 16));
    const float q = x * r;
    if (__builtin_expect(near_index_boundary(q), 0)) {
      const float v = x / s;
      b[j] = __builtin_isnan(v) ? uint32_t(kNan) : encode_q(v, lut);
    } else {
      b[j] = encode_q(q, lut);
    }
  }
  return make_uint2(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24), b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24));
}

// kQuant: also the static HiF8 codes of out with the fixed scale qs[0] (the
// next projection's input quant) and row_scale[row] = qs[0].
template <bool kResidual, bool kQuant = false>
__global__ __launch_bounds__(kRowThreads) void add_rms_norm_vec_kernel(uint16_t *__restrict__ h,
                                                                        const uint16_t *__restrict__ delta,
                                                                        const uint16_t *__restrict__ w,
                                                                        uint16_t *__restrict__ out, int n,
                                                                        float eps, const float *__restrict__ qs = nullptr,
                                                                        uint8_t *__restrict__ codes = nullptr,
                                                                        float *__restrict__ row_scale = nullptr) {
  __shared__ float red[kRowThreads / kWave];
  __shared__ __attribute__((aligned(16))) uint8_t lut[kQuant ? 8192 : 16];
  // The table copy is visible after the barriers of the row sum.
  if constexpr (kQuant) stage_static_encode_table(lut, threadIdx.x, kRowThreads);
  const int chunks = n / 8;
  uint4 *hr = reinterpret_cast<uint4 *>(h + size_t(blockIdx.x) * n);
  const uint4 *dr = kResidual ? reinterpret_cast<const uint4 *>(delta + size_t(blockIdx.x) * n) : nullptr;
  const uint4 *wr = reinterpret_cast<const uint4 *>(w);
  uint4 *orow = reinterpret_cast<uint4 *>(out + size_t(blockIdx.x) * n);
  uint4 hv[kRowChunks], dv[kRowChunks], wv[kRowChunks];
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = threadIdx.x + kRowThreads * c;
    if (i < chunks) {
      hv[c] = hr[i];
      if constexpr (kResidual) dv[c] = dr[i];
      wv[c] = wr[i];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = threadIdx.x + kRowThreads * c;
    if (i < chunks) {
      uint32_t hw[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float lo = __uint_as_float(hw[e] << 16), hi = __uint_as_float(hw[e] & 0xFFFF0000u);
        if constexpr (kResidual) {
          const uint32_t dw = e == 0 ? dv[c].x : e == 1 ? dv[c].y : e == 2 ? dv[c].z : dv[c].w;
          // the residual stream is bf16
          const uint32_t slo = to_bf(lo + __uint_as_float(dw << 16)), shi = to_bf(hi + __uint_as_float(dw & 0xFFFF0000u));
          hw[e] = slo | (shi << 16);
          lo = bf(uint16_t(slo));
          hi = bf(uint16_t(shi));
        }
        ss += lo * lo + hi * hi;
      }
      hv[c] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      if constexpr (kResidual) hr[i] = hv[c];
    }
  }
  const float r = rsqrtf(block_sum<kRowThreads>(ss, red) / float(n) + eps);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int i = threadIdx.x + kRowThreads * c;
    if (i < chunks) {
      const uint32_t hw[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
      const uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(hw[e] << 16) * r * __uint_as_float(ww[e] << 16);
        const float hi = __uint_as_float(hw[e] & 0xFFFF0000u) * r * __uint_as_float(ww[e] & 0xFFFF0000u);
        o[e] = uint32_t(to_bf(lo)) | (uint32_t(to_bf(hi)) << 16);
      }
      orow[i] = make_uint4(o[0], o[1], o[2], o[3]);
      if constexpr (kQuant)
        reinterpret_cast<uint2 *>(codes + size_t(blockIdx.x) * n)[i] = static_encode8(o, qs[0], lut);
    }
  }
  if (kQuant && threadIdx.x == 0) row_scale[blockIdx.x] = qs[0];
}

// SiLU-mul of rows of n % 8 == 0 straight to static HiF8 codes with the fixed
// scale qs[0] (the down projection's input quant): codes [rows, n] equal
// hif8_static_quant(hif8_silu_mul(gate_up)), row_scale[r] = qs[0].
__global__ __launch_bounds__(256) void silu_mul_quant_kernel(const uint16_t *__restrict__ gu,
                                                             const float *__restrict__ qs,
                                                             uint8_t *__restrict__ codes,
                                                             float *__restrict__ row_scale, int64_t rows, int n) {
  __shared__ __attribute__((aligned(16))) uint8_t lut[8192];
  stage_static_encode_table(lut, threadIdx.x, 256);
  __syncthreads();
  const float s = qs[0];
  const int groups = n / 8;
  const int64_t total = rows * groups;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t r = i / groups;
    const int c = int(i - r * groups);
    const uint4 g = *reinterpret_cast<const uint4 *>(gu + r * 2 * n + 8 * c);
    const uint4 u = *reinterpret_cast<const uint4 *>(gu + r * 2 * n + n + 8 * c);
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g0 = bf(uint16_t(gw[e])), g1 = bf(uint16_t(gw[e] >> 16));
      const float u0 = bf(uint16_t(uw[e])), u1 = bf(uint16_t(uw[e] >> 16));
      // the arithmetic of silu_mul_kernel, element by element
      o[e] = uint32_t(to_bf(g0 / (1.f + expf(-g0)) * u0)) | (uint32_t(to_bf(g1 / (1.f + expf(-g1)) * u1)) << 16);
    }
    reinterpret_cast<uint2 *>(codes + r * n)[c] = static_encode8(o, s, lut);
  }
  if (blockIdx.x == 0)
    for (int64_t r = threadIdx.x; r < rows; r += 256) row_scale[r] = s;
}

// out[m, n] = bf16(sum_k x[m, k] w[n, k]) for m < 4, bf16 operands, FP32
// accumulation: the small bf16 projections of the decode step (the
// linear-attention b/a projection, 2 * value heads outputs), which a library
// GEMM runs in ~14 us.  Block = kSmallRows output rows; thread t sums 16-byte
// chunks t, t + 256, ... of each; k % 8 == 0, 16-byte aligned rows.
// kSmallRows output rows per block: 4, or 1 for M >= 3 (more blocks for the
// few outputs: 64 x 4096 at M = 4 took 7.1 us with 4 rows per block).
// acc + the products of eight bf16 pairs (one 16-byte chunk of x and of a
// weight row), in the order every bf16 GEMV here sums them.
__device__ __forceinline__ float bf16_dot8(float acc, const uint4 xv, const uint4 wv) {
  const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    acc += __uint_as_float(xw[e] << 16) * __uint_as_float(ww[e] << 16) +
           __uint_as_float(xw[e] & 0xFFFF0000u) * __uint_as_float(ww[e] & 0xFFFF0000u);
  return acc;
}

template <int kM, int kSmallRows>
__global__ __launch_bounds__(kNormThreads) void bf16_gemv_kernel(const uint16_t *__restrict__ x,
                                                                 const uint16_t *__restrict__ w,
                                                                 uint16_t *__restrict__ out, int n, int k) {
  __shared__ float red[kNormThreads / kWave][kSmallRows * kM];
  const int n0 = blockIdx.x * kSmallRows, chunks = k / 8;
  float acc[kSmallRows][kM];
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r)
#pragma unroll
    for (int m = 0; m < kM; ++m) acc[r][m] = 0.f;
  for (int c = threadIdx.x; c < chunks; c += kNormThreads) {
    uint4 xv[kM], wv[kSmallRows];
#pragma unroll
    for (int m = 0; m < kM; ++m) xv[m] = reinterpret_cast<const uint4 *>(x + size_t(m) * k)[c];
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r)
      wv[r] = reinterpret_cast<const uint4 *>(w + size_t(min(n0 + r, n - 1)) * k)[c];
#pragma unroll
    for (int r = 0; r < kSmallRows; ++r)
#pragma unroll
      for (int m = 0; m < kM; ++m) acc[r][m] = bf16_dot8(acc[r][m], xv[m], wv[r]);
  }
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
#pragma unroll
  for (int r = 0; r < kSmallRows; ++r)
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      const float v = wave_sum(acc[r][m]);
      if (lane == 0) red[wave][r * kM + m] = v;
    }
  __syncthreads();
  if (threadIdx.x < kSmallRows * kM) {
    const int r = threadIdx.x / kM, m = threadIdx.x % kM;
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kNormThreads / kWave; ++i) v += red[i][threadIdx.x];
    if (n0 + r < n) out[size_t(m) * n + n0 + r] = to_bf(v);
  }
}

constexpr int kGdnThreads = 128;

// One block per (request, value head); thread j owns column j of the
// [dk, dv] state (dk, dv <= 128).
__global__ __launch_bounds__(kGdnThreads) void gdn_delta_kernel(
    const float *__restrict__ conv, int channels, const uint16_t *__restrict__ mixed, int64_t ld,
    const uint16_t *__restrict__ ba, const float *__restrict__ a_log, const float *__restrict__ dt_bias,
    float *__restrict__ state, const uint16_t *__restrict__ w_out, uint16_t *__restrict__ out, int k_heads,
    int v_heads, int dk, int dv, float eps) {
  __shared__ float qs[kGdnThreads], ks[kGdnThreads];
  __shared__ float red[kGdnThreads / kWave];
  const int b = blockIdx.x / v_heads, hv = blockIdx.x - b * v_heads;
  const int hk = hv / (v_heads / k_heads);
  const int qk_width = k_heads * dk;
  const int j = threadIdx.x;
  const float *cr = conv + size_t(b) * channels;
  const float qi = j < dk ? cr[hk * dk + j] : 0.f;
  const float ki = j < dk ? cr[qk_width + hk * dk + j] : 0.f;
  const float vj = j < dv ? cr[2 * qk_width + hv * dv + j] : 0.f;
  // F.normalize: x / max(||x||, 1e-12); q also scaled by 1 / sqrt(dk).
  const float qn = fmaxf(sqrtf(block_sum<kGdnThreads>(qi * qi, red)), 1e-12f);
  const float kn = fmaxf(sqrtf(block_sum<kGdnThreads>(ki * ki, red)), 1e-12f);
  const float qv = qi / qn / sqrtf(float(dk)), kv = ki / kn;
  qs[j] = qv;
  ks[j] = kv;
  const float kq = block_sum<kGdnThreads>(kv * qv, red);  // also orders the qs / ks stores
  const float braw = bf(ba[size_t(b) * 2 * v_heads + hv]);
  const float araw = bf(ba[size_t(b) * 2 * v_heads + v_heads + hv]) + dt_bias[hv];
  const float beta = 1.f / (1.f + expf(-braw));
  const float softplus = araw > 20.f ? araw : log1pf(expf(araw));
  const float decay = expf(-expf(a_log[hv]) * softplus);
  float *S = state + (size_t(b) * v_heads + hv) * dk * dv;
  float o = 0.f;
  if (j < dv) {
    float a = 0.f, c = 0.f;
    for (int i = 0; i < dk; ++i) {
      const float s = S[size_t(i) * dv + j];
      a += s * ks[i];
      c += s * qs[i];
    }
    const float delta = beta * (vj - decay * a);
    o = decay * c + delta * kq;
    for (int i = 0; i < dk; ++i) {
      float *p = S + size_t(i) * dv + j;
      *p = decay * *p + ks[i] * delta;
    }
  }
  const float r = rsqrtf(block_sum<kGdnThreads>(j < dv ? o * o : 0.f, red) / float(dv) + eps);
  if (j < dv) {
    const float z = bf(mixed[size_t(b) * ld + 2 * qk_width + v_heads * dv + hv * dv + j]);
    out[(size_t(b) * v_heads + hv) * dv + j] = to_bf(o * r * bf(w_out[j]) * (z / (1.f + expf(-z))));
  }
}

// The same step with each (request, value head) spread over 1024 threads:
// thread (part, j) owns rows [part * R, part * R + R) of state column j
// (R = dk / 8 <= 16), loads them at once and keeps them in registers; the
// column sums S^T k and S^T q meet in LDS.  One block per head with 128
// threads walking all dk rows twice took ~33 us per layer (dk = dv = 128).
// Requires dk % 8 == 0, dk <= 128, dv <= 128.
constexpr int kGdnParts = 8, kGdnCols = 128, kGdnWideThreads = kGdnParts * kGdnCols;
constexpr int kGdnRows = 16;  // rows per part, at most

__global__ __launch_bounds__(kGdnWideThreads) void gdn_delta_wide_kernel(
    const float *__restrict__ conv, int channels, const uint16_t *__restrict__ mixed, int64_t ld,
    const uint16_t *__restrict__ ba, const float *__restrict__ a_log, const float *__restrict__ dt_bias,
    float *__restrict__ state, const uint16_t *__restrict__ w_out, uint16_t *__restrict__ out, int k_heads,
    int v_heads, int dk, int dv, float eps) {
  __shared__ float qs[kGdnCols], ks[kGdnCols];
  __shared__ float pa[kGdnParts][kGdnCols], pc[kGdnParts][kGdnCols];
  __shared__ float red[kGdnWideThreads / kWave];
  const int b = blockIdx.x / v_heads, hv = blockIdx.x - b * v_heads;
  const int hk = hv / (v_heads / k_heads);
  const int qk_width = k_heads * dk;
  const int j = threadIdx.x % kGdnCols, part = threadIdx.x / kGdnCols;
  const int rows = dk / kGdnParts, r0 = part * rows;
  const bool col_ok = j < dv;
  float *S = state + (size_t(b) * v_heads + hv) * dk * dv;
  // State rows first (the longest loads), then the conv outputs.
  float sv[kGdnRows];
#pragma unroll
  for (int i = 0; i < kGdnRows; ++i) sv[i] = (i < rows && col_ok) ? S[size_t(r0 + i) * dv + j] : 0.f;
  const float *cr = conv + size_t(b) * channels;
  const bool lead = part == 0;
  const float qi = lead && j < dk ? cr[hk * dk + j] : 0.f;
  const float ki = lead && j < dk ? cr[qk_width + hk * dk + j] : 0.f;
  const float vj = col_ok ? cr[2 * qk_width + hv * dv + j] : 0.f;
  // F.normalize: x / max(||x||, 1e-12); q also scaled by 1 / sqrt(dk).
  const float qn = fmaxf(sqrtf(block_sum<kGdnWideThreads>(qi * qi, red)), 1e-12f);
  const float kn = fmaxf(sqrtf(block_sum<kGdnWideThreads>(ki * ki, red)), 1e-12f);
  const float qv = qi / qn / sqrtf(float(dk)), kv = ki / kn;
  if (lead) {
    qs[j] = qv;
    ks[j] = kv;
  }
  const float kq = block_sum<kGdnWideThreads>(kv * qv, red);  // also orders the qs / ks stores
  const float braw = bf(ba[size_t(b) * 2 * v_heads + hv]);
  const float araw = bf(ba[size_t(b) * 2 * v_heads + v_heads + hv]) + dt_bias[hv];
  const float beta = 1.f / (1.f + expf(-braw));
  const float softplus = araw > 20.f ? araw : log1pf(expf(araw));
  const float decay = expf(-expf(a_log[hv]) * softplus);
  float a = 0.f, c = 0.f;
#pragma unroll
  for (int i = 0; i < kGdnRows; ++i) {
    if (i < rows) {
      a += sv[i] * ks[r0 + i];
      c += sv[i] * qs[r0 + i];
    }
  }
  pa[part][j] = a;
  pc[part][j] = c;
  __syncthreads();
  a = 0.f;
  c = 0.f;
#pragma unroll
  for (int p = 0; p < kGdnParts; ++p) {
    a += pa[p][j];
    c += pc[p][j];
  }
  const float delta = beta * (vj - decay * a);
  const float o = decay * c + delta * kq;
  if (col_ok) {
#pragma unroll
    for (int i = 0; i < kGdnRows; ++i)
      if (i < rows) S[size_t(r0 + i) * dv + j] = decay * sv[i] + ks[r0 + i] * delta;
  }
  const float r = rsqrtf(block_sum<kGdnWideThreads>(lead && col_ok ? o * o : 0.f, red) / float(dv) + eps);
  if (lead && col_ok) {
    const float z = bf(mixed[size_t(b) * ld + 2 * qk_width + v_heads * dv + hv * dv + j]);
    out[(size_t(b) * v_heads + hv) * dv + j] = to_bf(o * r * bf(w_out[j]) * (z / (1.f + expf(-z))));
  }
}

// One decode token of the linear-attention mixer for the value heads of KV
// group (request b, key head hk), fused with the b/a projection and the conv:
// the kRep = v_heads / k_heads value heads of the group share its q and k, so
// the block owns every conv channel it reads (q and k of hk, v of its value
// heads) and shifts that channel's state alone.  The kRep heads run side by
// side, each on 1024 / kRep threads: thread (head, part, j) owns rows
// [part * R, part * R + R) of state column j, R = dk * kRep / 8 (<= 32),
// loaded at kernel entry into registers.  Four barriers in all: after the
// conv and the b/a row sums (one 256-thread team per row, as hif8_bf16_gemv
// sums a row, so b and a round to the same bf16 values); after the q / k
// sums (|q|^2, |k|^2 and q.k from the raw conv outputs in one pass; the
// normalisation is applied to the dot products afterwards, S^T k = (S^T
// k_raw) / |k|, so only one reduction precedes the state dot products);
// after the column partials of S^T k and S^T q; after the output norm.  The
// b/a values equal hif8_bf16_gemv's bit for bit; the state and output agree
// with hif8_gdn_decode_step to FP32 rounding (the dot products are scaled
// after the sum instead of before).  Requires kRep <= 2, dk % 8 == 0,
// dk <= 128, dv <= 128, 2 dk + kRep dv <= 1024, hidden % 8 == 0,
// hidden <= 8192.
template <int kRep, int kKw>
__global__ __launch_bounds__(kGdnWideThreads) void gdn_token_kernel(
    const uint16_t *__restrict__ mixed, int64_t ld, const uint16_t *__restrict__ x,
    const uint16_t *__restrict__ w_ba, int hidden, const uint16_t *__restrict__ conv_w,
    uint16_t *__restrict__ conv_state, const float *__restrict__ a_log, const float *__restrict__ dt_bias,
    float *__restrict__ state, const uint16_t *__restrict__ w_out, uint16_t *__restrict__ out, int k_heads,
    int v_heads, int dk, int dv, float eps) {
  static_assert(kRep >= 1 && kRep <= 2, "one or two value heads per key head");
  constexpr int kHeadT = kGdnWideThreads / kRep;  // threads per value head
  constexpr int kParts = kHeadT / kGdnCols;       // row parts per head
  constexpr int kRows = kGdnRows * kRep;          // rows per part, at most
  // Conv outputs: q | k | v of each value head, then one slot per other
  // thread (every thread stores its conv, so its loads issue first).
  __shared__ float cbuf[kGdnWideThreads];
  __shared__ float pa[kRep][kParts][kGdnCols], pc[kRep][kParts][kGdnCols];
  __shared__ float ba_red[2 * kRep][kNormThreads / kWave];
  __shared__ float qk_red[2][3];                 // waves 0-1: |q|^2, |k|^2, q.k
  __shared__ float o_red[kRep][2];               // the two lead waves of each head: |o|^2
  const int b = blockIdx.x / k_heads, hk = blockIdx.x - b * k_heads;
  const int qk_width = k_heads * dk, channels = 2 * qk_width + v_heads * dv;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int head = tid / kHeadT, ht = tid % kHeadT;
  const int j = ht % kGdnCols, part = ht / kGdnCols;
  const int rows = dk / kParts, r0 = part * rows;
  const bool col_ok = j < dv;
  const int hv = kRep * hk + head;
  // Every load is issued up front, in the order the values are consumed:
  // the conv inputs, the b/a chunks, the state rows, the output-gate values.
  // Conv thread t < nch owns channel q[t] of hk, then k of hk, then v of the
  // value heads.
  const int nch = 2 * dk + kRep * dv;
  const bool conv_thread = tid < nch;
  const int cch = !conv_thread     ? 0
                  : tid < dk       ? hk * dk + tid
                  : tid < 2 * dk   ? qk_width + hk * dk + (tid - dk)
                                   : 2 * qk_width + kRep * hk * dv + (tid - 2 * dk);
  // Loads take clamped indices instead of predicates and land in 32-bit
  // registers, so they issue back to back with no wait between them; lanes
  // and taps past the end read in-bounds values they ignore.
  uint16_t *cst = conv_state + (size_t(b) * channels + cch) * (kKw - 1);
  uint32_t stv[kKw - 1], cwv[kKw];
  const uint32_t xc = mixed[size_t(b) * ld + cch];
#pragma unroll
  for (int t = 0; t < kKw - 1; ++t) stv[t] = cst[t];
#pragma unroll
  for (int t = 0; t < kKw; ++t) cwv[t] = conv_w[size_t(cch) * kKw + t];
  // b/a projection: team t (256 threads) sums row b (t even) or a (t odd) of
  // value head t / 2.
  const int team = tid / kNormThreads, tt = tid % kNormThreads;
  constexpr int kMaxChunks = 4;  // hidden <= 8 * 256 * 4
  uint4 xv[kMaxChunks], wv[kMaxChunks];
  const int chunks = hidden / 8;
  if (team < 2 * kRep) {
    const int hvt = kRep * hk + team / 2;
    const uint4 *wr = reinterpret_cast<const uint4 *>(w_ba + size_t(team % 2 ? v_heads + hvt : hvt) * hidden);
    const uint4 *xr = reinterpret_cast<const uint4 *>(x + size_t(b) * hidden);
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      const int i = min(tt + kNormThreads * c, chunks - 1);
      xv[c] = xr[i];
      wv[c] = wr[i];
    }
  }
  float sv[kRows];
  {
    const float *S = state + (size_t(b) * v_heads + hv) * dk * dv;
#pragma unroll
    for (int r = 0; r < kRows; ++r) sv[r] = S[size_t(r0 + min(r, rows - 1)) * dv + min(j, dv - 1)];
  }
  const bool lead = part == 0;
  const uint32_t zraw = mixed[size_t(b) * ld + 2 * qk_width + v_heads * dv + hv * dv + min(j, dv - 1)];
  const uint32_t wo = w_out[min(j, dv - 1)];
  const float dtb = dt_bias[hv], alog = a_log[hv];
  // Conv, as gdn_conv_kernel, on every thread; the conv threads shift the
  // channel's state by one.
  float cacc = 0.f;
#pragma unroll
  for (int t = 0; t < kKw - 1; ++t) cacc += bf(stv[t]) * bf(cwv[t]);
  cacc += bf(xc) * bf(cwv[kKw - 1]);
  cbuf[tid] = cacc / (1.f + expf(-cacc));
  if (conv_thread) {
#pragma unroll
    for (int t = 0; t + 1 < kKw - 1; ++t) cst[t] = uint16_t(stv[t + 1]);
    cst[kKw - 2] = uint16_t(xc);
  }
  if (team < 2 * kRep) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c)
      if (tt + kNormThreads * c < chunks) acc = bf16_dot8(acc, xv[c], wv[c]);
    const float v = wave_sum(acc);
    if (lane == 0) ba_red[team][tt / kWave] = v;
  }
  __syncthreads();
  // |q|^2, |k|^2 and q.k over the dk channels (waves 0 and 1: threads 0..127).
  if (wave < 2) {
    const float qi = tid < dk ? cbuf[tid] : 0.f, ki = tid < dk ? cbuf[dk + tid] : 0.f;
    const float s0 = wave_sum(qi * qi), s1 = wave_sum(ki * ki), s2 = wave_sum(qi * ki);
    if (lane == 0) {
      qk_red[wave][0] = s0;
      qk_red[wave][1] = s1;
      qk_red[wave][2] = s2;
    }
  }
  // Column partials of S^T k_raw and S^T q_raw over this part's rows.
  float a = 0.f, c = 0.f;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    if (r < rows) {
      a += sv[r] * cbuf[dk + r0 + r];
      c += sv[r] * cbuf[r0 + r];
    }
  }
  pa[head][part][j] = a;
  pc[head][part][j] = c;
  __syncthreads();
  // F.normalize: x / max(||x||, 1e-12); q also scaled by 1 / sqrt(dk).
  const float qn = fmaxf(sqrtf(qk_red[0][0] + qk_red[1][0]), 1e-12f);
  const float kn = fmaxf(sqrtf(qk_red[0][1] + qk_red[1][1]), 1e-12f);
  const float qscale = 1.f / qn / sqrtf(float(dk)), kscale = 1.f / kn;
  const float kq = (qk_red[0][2] + qk_red[1][2]) * qscale * kscale;
  a = 0.f;
  c = 0.f;
#pragma unroll
  for (int p = 0; p < kParts; ++p) {
    a += pa[head][p][j];
    c += pc[head][p][j];
  }
  a *= kscale;
  c *= qscale;
  float bsum = 0.f, asum = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) {
    bsum += ba_red[2 * head][w];
    asum += ba_red[2 * head + 1][w];
  }
  const float braw = bf(to_bf(bsum));
  const float araw = bf(to_bf(asum)) + dtb;
  const float vj = col_ok ? cbuf[2 * dk + head * dv + j] : 0.f;
  const float beta = 1.f / (1.f + expf(-braw));
  const float softplus = araw > 20.f ? araw : log1pf(expf(araw));
  const float decay = expf(-expf(alog) * softplus);
  const float delta = beta * (vj - decay * a);
  const float o = decay * c + delta * kq;
  if (col_ok) {
    float *S = state + (size_t(b) * v_heads + hv) * dk * dv;
#pragma unroll
    for (int r = 0; r < kRows; ++r)
      if (r < rows) S[size_t(r0 + r) * dv + j] = decay * sv[r] + cbuf[dk + r0 + r] * kscale * delta;
  }
  // Output RMSNorm over the head's dv columns (the part-0 threads of the
  // head: its first two wavefronts).
  const int hw = ht / kWave;  // wavefront within the head
  if (hw < 2) {
    const float v = wave_sum(lead && col_ok ? o * o : 0.f);
    if (lane == 0) o_red[head][hw] = v;
  }
  __syncthreads();
  if (lead && col_ok) {
    const float rn = rsqrtf((o_red[head][0] + o_red[head][1]) / float(dv) + eps);
    const float z = bf(zraw);
    out[(size_t(b) * v_heads + hv) * dv + j] = to_bf(o * rn * bf(wo) * (z / (1.f + expf(-z))));
  }
}

// One decode token of the linear-attention recurrence for one (request b,
// value head hv), from conv [b, channels] (fp32, SiLU applied: q | k | v, as
// the qkvz projection's conv epilogue writes them), fused with the b/a
// projection of the head.  Thread (part, j) owns rows [part * kR, part * kR +
// kR) of state column j (dk = 8 kR), loaded at kernel entry into registers
// with every other load.  Three barriers: after the b/a row sums (two
// 256-thread teams, as hif8_bf16_gemv sums a row, so b and a round to its bf16
// values) and the q / k sums (|q|^2, |k|^2 and q.k over the raw conv outputs;
// S^T k = (S^T k_raw) / |k|, S^T q likewise, so one reduction precedes the
// state dot products); after the column partials; after the output norm.
// The arithmetic per head is gdn_token_kernel's.  One head per block spreads
// a step over batch * v_heads blocks where the group kernel puts two heads'
// 32768 state elements on one CU, whose VALU then bounds it: on MI355X at
// b = 1 (16 key heads, 32 value heads, dk = dv = 128) 6.8 us per call in the
// decode step's kernel trace against 12.5 us for the group kernel.  Requires
// dk = 8 kR, dv <= 128, hidden % 8 == 0, hidden <= 8192.
template <int kR>
__global__ __launch_bounds__(kGdnWideThreads) void gdn_head_kernel(
    const float *__restrict__ conv, const uint16_t *__restrict__ mixed, int64_t ld, const uint16_t *__restrict__ x,
    const uint16_t *__restrict__ w_ba, int hidden, const float *__restrict__ a_log,
    const float *__restrict__ dt_bias, float *__restrict__ state, const uint16_t *__restrict__ w_out,
    uint16_t *__restrict__ out, int k_heads, int v_heads, int dv, float eps) {
  constexpr int dk = kGdnParts * kR;
  __shared__ __attribute__((aligned(16))) float qs[dk], ks[dk];  // raw conv outputs of q and k
  __shared__ float pa[kGdnParts][kGdnCols], pc[kGdnParts][kGdnCols];
  __shared__ float ba_red[2][kNormThreads / kWave];
  __shared__ float qk_red[2][3];  // waves 0-1: |q|^2, |k|^2, q.k
  __shared__ float o_red[2];      // waves 0-1: |o|^2
  const int b = blockIdx.x / v_heads, hv = blockIdx.x - b * v_heads;
  const int hk = hv / (v_heads / k_heads);
  const int qk_width = k_heads * dk, channels = 2 * qk_width + v_heads * dv;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int j = tid % kGdnCols, part = tid / kGdnCols, r0 = part * kR;
  const bool col_ok = j < dv;
  const int jc = min(j, dv - 1);
  // Every load first, with clamped indices (no predicates, so they issue
  // back to back; lanes past the end read in-bounds values they ignore).
  const float *cr = conv + size_t(b) * channels;
  const int qt = min(tid, dk - 1);
  const float qraw = cr[hk * dk + qt], kraw = cr[qk_width + hk * dk + qt];
  const int team = tid / kNormThreads, tt = tid % kNormThreads;
  constexpr int kMaxChunks = 4;  // hidden <= 8 * 256 * 4
  uint4 xv[kMaxChunks], wv[kMaxChunks];
  const int chunks = hidden / 8;
  if (team < 2) {
    const uint4 *wr = reinterpret_cast<const uint4 *>(w_ba + size_t(team ? v_heads + hv : hv) * hidden);
    const uint4 *xr = reinterpret_cast<const uint4 *>(x + size_t(b) * hidden);
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      const int i = min(tt + kNormThreads * c, chunks - 1);
      xv[c] = xr[i];
      wv[c] = wr[i];
    }
  }
  float *S = state + (size_t(b) * v_heads + hv) * dk * dv;
  float sv[kR];
#pragma unroll
  for (int r = 0; r < kR; ++r) sv[r] = S[size_t(r0 + r) * dv + jc];
  const float vj = cr[2 * qk_width + hv * dv + jc];
  const uint32_t zraw = mixed[size_t(b) * ld + 2 * qk_width + v_heads * dv + hv * dv + jc];
  const uint32_t wo = w_out[jc];
  const float dtb = dt_bias[hv], alog = a_log[hv];
  if (tid < dk) {
    qs[tid] = qraw;
    ks[tid] = kraw;
  }
  if (wave < 2) {
    const float qi = tid < dk ? qraw : 0.f, ki = tid < dk ? kraw : 0.f;
    const float s0 = wave_sum(qi * qi), s1 = wave_sum(ki * ki), s2 = wave_sum(qi * ki);
    if (lane == 0) {
      qk_red[wave][0] = s0;
      qk_red[wave][1] = s1;
      qk_red[wave][2] = s2;
    }
  }
  if (team < 2) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c)
      if (tt + kNormThreads * c < chunks) acc = bf16_dot8(acc, xv[c], wv[c]);
    const float v = wave_sum(acc);
    if (lane == 0) ba_red[team][tt / kWave] = v;
  }
  __syncthreads();
  // Column partials of S^T k_raw and S^T q_raw over this part's rows.
  float a = 0.f, c = 0.f;
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    a += sv[r] * ks[r0 + r];
    c += sv[r] * qs[r0 + r];
  }
  pa[part][j] = a;
  pc[part][j] = c;
  __syncthreads();
  // F.normalize: x / max(||x||, 1e-12); q also scaled by 1 / sqrt(dk).
  const float qn = fmaxf(sqrtf(qk_red[0][0] + qk_red[1][0]), 1e-12f);
  const float kn = fmaxf(sqrtf(qk_red[0][1] + qk_red[1][1]), 1e-12f);
  const float qscale = 1.f / qn / sqrtf(float(dk)), kscale = 1.f / kn;
  const float kq = (qk_red[0][2] + qk_red[1][2]) * qscale * kscale;
  a = 0.f;
  c = 0.f;
#pragma unroll
  for (int p = 0; p < kGdnParts; ++p) {
    a += pa[p][j];
    c += pc[p][j];
  }
  a *= kscale;
  c *= qscale;
  float bsum = 0.f, asum = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) {
    bsum += ba_red[0][w];
    asum += ba_red[1][w];
  }
  const float braw = bf(to_bf(bsum));
  const float araw = bf(to_bf(asum)) + dtb;
  const float beta = 1.f / (1.f + expf(-braw));
  const float softplus = araw > 20.f ? araw : log1pf(expf(araw));
  const float decay = expf(-expf(alog) * softplus);
  const float delta = beta * ((col_ok ? vj : 0.f) - decay * a);
  const float o = decay * c + delta * kq;
  if (col_ok) {
#pragma unroll
    for (int r = 0; r < kR; ++r) S[size_t(r0 + r) * dv + j] = decay * sv[r] + ks[r0 + r] * kscale * delta;
  }
  // Output RMSNorm over the dv columns (the part-0 threads: waves 0-1).
  if (wave < 2) {
    const float v = wave_sum(col_ok ? o * o : 0.f);
    if (lane == 0) o_red[wave] = v;
  }
  __syncthreads();
  if (part == 0 && col_ok) {
    const float rn = rsqrtf((o_red[0] + o_red[1]) / float(dv) + eps);
    const float z = bf(uint16_t(zraw));
    out[(size_t(b) * v_heads + hv) * dv + j] = to_bf(o * rn * bf(uint16_t(wo)) * (z / (1.f + expf(-z))));
  }
}

constexpr int kHeadThreads = 256;

// One block per (request, head of q | k | v) of a decode token: q and k heads
// RMS-normalised (weight w_q / w_k) and rotated on their first rot dims
// (halves i, i + rot/2, angle pos * inv_freq[i]); v heads copied.  Block
// (b, 0) also writes the cache slot of position pos[b].
__global__ __launch_bounds__(kHeadThreads) void qk_norm_rope_kernel(
    const uint16_t *__restrict__ qkv, const uint16_t *__restrict__ w_q, const uint16_t *__restrict__ w_k,
    const int64_t *__restrict__ pos, const float *__restrict__ inv_freq, const int32_t *__restrict__ block_table,
    int64_t max_blocks, int block_size, uint16_t *__restrict__ q_out, uint16_t *__restrict__ k_out,
    uint16_t *__restrict__ v_out, int64_t *__restrict__ slots, int hq, int hkv, int d, int rot, float eps) {
  __shared__ float y[kHeadThreads];
  __shared__ float red[kHeadThreads / kWave];
  const int heads = hq + 2 * hkv;
  const int b = blockIdx.x / heads, h = blockIdx.x - b * heads;
  const int j = threadIdx.x;
  const float x = j < d ? bf(qkv[(size_t(b) * heads + h) * d + j]) : 0.f;
  const int64_t p = pos[b];
  if (h == 0 && j == 0 && slots) {
    // A position outside the table (negative, or past max_blocks pages, e.g.
    // a replayed graph run past its capacity) gets slot -1, which the cache
    // write skips as padding; the table is never read out of bounds.
    int64_t slot = -1;
    if (p >= 0 && p / block_size < max_blocks) {
      const int64_t blk = block_table[size_t(b) * max_blocks + p / block_size];
      if (blk >= 0) slot = blk * block_size + p % block_size;
    }
    slots[b] = slot;
  }
  if (h >= hq + hkv) {
    if (j < d) v_out[(size_t(b) * hkv + (h - hq - hkv)) * d + j] = qkv[(size_t(b) * heads + h) * d + j];
    return;
  }
  const bool is_q = h < hq;
  const float r = rsqrtf(block_sum<kHeadThreads>(x * x, red) / float(d) + eps);
  const float yn = j < d ? bf(to_bf(x * r * bf((is_q ? w_q : w_k)[j]))) : 0.f;  // the normed head is bf16
  y[j] = yn;
  __syncthreads();
  float out = yn;
  if (j < rot) {
    const int half = rot / 2, i = j < half ? j : j - half;
    const float ang = float(p) * inv_freq[i];
    const float c = cosf(ang), s = sinf(ang);
    out = j < half ? y[j] * c - y[j + half] * s : y[j] * c + y[j - half] * s;
  }
  if (j < d) {
    uint16_t *dst = is_q ? q_out + (size_t(b) * hq + h) * d : k_out + (size_t(b) * hkv + (h - hq)) * d;
    dst[j] = to_bf(out);
  }
}

}  // namespace
}  // namespace hif8

using namespace hif8;

extern "C" int hif8_qk_norm_rope(const uint16_t *qkv, const uint16_t *q_norm, const uint16_t *k_norm,
                                 const int64_t *pos, const float *inv_freq, const int32_t *block_table,
                                 int64_t max_blocks, int64_t block_size, uint16_t *q_out, uint16_t *k_out,
                                 uint16_t *v_out, int64_t *slots, int64_t batch, int64_t num_heads,
                                 int64_t num_kv_heads, int64_t head_size, int64_t rotary_dim, float eps,
                                 hif8_stream_t stream) {
  clear_error();
  if (!qkv || !q_norm || !k_norm || !pos || !inv_freq || !q_out || !k_out || !v_out || (slots && !block_table))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_qk_norm_rope: null pointer argument");
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 || head_size > kHeadThreads ||
      rotary_dim < 0 || rotary_dim > head_size || rotary_dim % 2 || block_size <= 0 || batch > 65536)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_qk_norm_rope: unsupported dimensions");
  qk_norm_rope_kernel<<<unsigned(batch * (num_heads + 2 * num_kv_heads)), kHeadThreads, 0,
                        reinterpret_cast<hipStream_t>(stream)>>>(
      qkv, q_norm, k_norm, pos, inv_freq, block_table, max_blocks, int(block_size), q_out, k_out, v_out, slots,
      int(num_heads), int(num_kv_heads), int(head_size), int(rotary_dim), eps);
  return check_launch("hif8_qk_norm_rope");
}

extern "C" int hif8_add_rms_norm(uint16_t *h, const uint16_t *delta, const uint16_t *weight, uint16_t *out,
                                 int64_t rows, int64_t n, float eps, hif8_stream_t stream) {
  clear_error();
  if (!h || !weight || !out) return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_add_rms_norm: null pointer argument");
  if (rows <= 0 || n <= 0 || rows > 0x7FFFFFFFll || n > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_add_rms_norm: invalid dimensions");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = n % 8 == 0 && n <= 8 * kRowThreads * kRowChunks && aligned(h, 16) && aligned(weight, 16) &&
                   aligned(out, 16) && (!delta || aligned(delta, 16));
  if (vec && delta)
    add_rms_norm_vec_kernel<true><<<unsigned(rows), kRowThreads, 0, s>>>(h, delta, weight, out, int(n), eps);
  else if (vec)
    add_rms_norm_vec_kernel<false><<<unsigned(rows), kRowThreads, 0, s>>>(h, nullptr, weight, out, int(n), eps);
  else if (delta)
    add_rms_norm_kernel<true><<<unsigned(rows), kNormThreads, 0, s>>>(h, delta, weight, out, int(n), eps);
  else
    add_rms_norm_kernel<false><<<unsigned(rows), kNormThreads, 0, s>>>(h, nullptr, weight, out, int(n), eps);
  return check_launch("hif8_add_rms_norm");
}

extern "C" int hif8_add_rms_norm_quant(uint16_t *h, const uint16_t *delta, const uint16_t *weight, uint16_t *out,
                                       const float *input_scale, uint8_t *codes, float *row_scale, int64_t rows,
                                       int64_t n, float eps, hif8_stream_t stream) {
  clear_error();
  if (!h || !weight || !out || !input_scale || !codes || !row_scale)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_add_rms_norm_quant: null pointer argument");
  if (rows <= 0 || n <= 0 || rows > 0x7FFFFFFFll || n > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_add_rms_norm_quant: invalid dimensions");
  if (n % 8 || n > 8 * kRowThreads * kRowChunks || !aligned(h, 16) || !aligned(weight, 16) || !aligned(out, 16) ||
      (delta && !aligned(delta, 16)) || !aligned(codes, 8))
    return fail(HIF8_ERR_UNSUPPORTED, "hif8_add_rms_norm_quant: needs n %% 8 == 0, n <= %d and aligned rows",
                8 * kRowThreads * kRowChunks);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (delta)
    add_rms_norm_vec_kernel<true, true><<<unsigned(rows), kRowThreads, 0, s>>>(h, delta, weight, out, int(n), eps,
                                                                               input_scale, codes, row_scale);
  else
    add_rms_norm_vec_kernel<false, true><<<unsigned(rows), kRowThreads, 0, s>>>(h, nullptr, weight, out, int(n), eps,
                                                                                input_scale, codes, row_scale);
  return check_launch("hif8_add_rms_norm_quant");
}

extern "C" int hif8_silu_mul_quant(const uint16_t *gate_up, const float *input_scale, uint8_t *codes,
                                   float *row_scale, int64_t rows, int64_t n, hif8_stream_t stream) {
  clear_error();
  if (!gate_up || !input_scale || !codes || !row_scale)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_silu_mul_quant: null pointer argument");
  if (rows <= 0 || n <= 0 || n > 0x7FFFFFFFll || rows > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_silu_mul_quant: invalid dimensions");
  if (n % 8 || !aligned(gate_up, 16) || !aligned(codes, 8))
    return fail(HIF8_ERR_UNSUPPORTED, "hif8_silu_mul_quant: needs n %% 8 == 0 and aligned rows");
  const int64_t blocks = std::min<int64_t>((rows * (n / 8) + 255) / 256, 4096);
  silu_mul_quant_kernel<<<unsigned(blocks), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      gate_up, input_scale, codes, row_scale, rows, int(n));
  return check_launch("hif8_silu_mul_quant");
}

extern "C" int hif8_silu_mul(const uint16_t *gate_up, uint16_t *out, int64_t rows, int64_t n, hif8_stream_t stream) {
  clear_error();
  if (!gate_up || !out) return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_silu_mul: null pointer argument");
  if (rows <= 0 || n <= 0 || n > 0x7FFFFFFFll) return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_silu_mul: invalid dimensions");
  const int64_t blocks = std::min<int64_t>((rows * n + 255) / 256, 4096);
  silu_mul_kernel<<<unsigned(blocks), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(gate_up, out, rows, int(n));
  return check_launch("hif8_silu_mul");
}

extern "C" int hif8_bf16_gemv(const uint16_t *x, const uint16_t *weight, uint16_t *out, int64_t m, int64_t n,
                              int64_t k, hif8_stream_t stream) {
  clear_error();
  if (!x || !weight || !out) return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_bf16_gemv: null pointer argument");
  if (m < 1 || m > 4 || n <= 0 || k <= 0 || n > 0x7FFFFFFFll || k > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_bf16_gemv: needs 1 <= M <= 4 and positive N, K");
  if (k % 8 || !aligned(x, 16) || !aligned(weight, 16))
    return fail(HIF8_ERR_UNSUPPORTED, "hif8_bf16_gemv: needs K %% 8 == 0 and 16-byte aligned operands");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid4{unsigned((n + 3) / 4)}, grid1{unsigned(n)};
  switch (m) {
    case 1: bf16_gemv_kernel<1, 4><<<grid4, kNormThreads, 0, s>>>(x, weight, out, int(n), int(k)); break;
    case 2: bf16_gemv_kernel<2, 4><<<grid4, kNormThreads, 0, s>>>(x, weight, out, int(n), int(k)); break;
    // One row per block for M >= 3 gives a short output more blocks; from
    // 4096 outputs on, four rows per block stream the weight faster (an LM
    // head, 151936 x 4096 at M = 4: 353 us with one row per block).
    case 3:
      if (n >= 4096) bf16_gemv_kernel<3, 4><<<grid4, kNormThreads, 0, s>>>(x, weight, out, int(n), int(k));
      else bf16_gemv_kernel<3, 1><<<grid1, kNormThreads, 0, s>>>(x, weight, out, int(n), int(k));
      break;
    default:
      if (n >= 4096) bf16_gemv_kernel<4, 4><<<grid4, kNormThreads, 0, s>>>(x, weight, out, int(n), int(k));
      else bf16_gemv_kernel<4, 1><<<grid1, kNormThreads, 0, s>>>(x, weight, out, int(n), int(k));
      break;
  }
  return check_launch("hif8_bf16_gemv");
}

extern "C" int hif8_gdn_decode_token(const uint16_t *mixed_qkvz, int64_t ld, const uint16_t *x,
                                     const uint16_t *ba_weight, int64_t hidden, const uint16_t *conv_weight,
                                     uint16_t *conv_state, const float *a_log, const float *dt_bias,
                                     float *rec_state, const uint16_t *out_norm, uint16_t *out, int64_t batch,
                                     int64_t k_heads, int64_t v_heads, int64_t k_dim, int64_t v_dim,
                                     int64_t conv_width, float eps, hif8_stream_t stream) {
  clear_error();
  if (!mixed_qkvz || !x || !ba_weight || !conv_weight || !conv_state || !a_log || !dt_bias || !rec_state ||
      !out_norm || !out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_token: null pointer argument");
  if (batch <= 0 || k_heads <= 0 || v_heads <= 0 || v_heads % k_heads || k_dim <= 0 || v_dim <= 0 ||
      hidden <= 0 || hidden > 0x7FFFFFFFll || conv_width < 2 || conv_width > 16 || batch * k_heads > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_token: unsupported dimensions");
  const int64_t channels = 2 * k_heads * k_dim + v_heads * v_dim;
  if (ld < channels + v_heads * v_dim)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_token: mixed_qkvz row too short");
  const int64_t rep = v_heads / k_heads;
  if (rep > 2 || k_dim % kGdnParts || k_dim > kGdnParts * kGdnRows || v_dim > kGdnCols ||
      2 * k_dim + rep * v_dim > kGdnWideThreads || hidden % 8 || hidden > 8 * kNormThreads * 4 ||
      conv_width > 4 ||
      !aligned(x, 16) || !aligned(ba_weight, 16))
    return fail(HIF8_ERR_UNSUPPORTED, "hif8_gdn_decode_token: needs v_heads / k_heads <= 2, k_dim %% 8 == 0, "
                                      "k_dim, v_dim <= 128, hidden %% 8 == 0, hidden <= 8192, conv_width <= 4 "
                                      "and 16-byte aligned x / ba_weight");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(unsigned(batch * k_heads));
#define HIF8_GDN_TOKEN(R, W)                                                                                     \
  gdn_token_kernel<R, W><<<grid, kGdnWideThreads, 0, s>>>(mixed_qkvz, ld, x, ba_weight, int(hidden), conv_weight, \
                                                          conv_state, a_log, dt_bias, rec_state, out_norm, out,      \
                                                          int(k_heads), int(v_heads), int(k_dim), int(v_dim), eps)
#define HIF8_GDN_TOKEN_W(R)             \
  switch (conv_width) {                 \
    case 2: HIF8_GDN_TOKEN(R, 2); break; \
    case 3: HIF8_GDN_TOKEN(R, 3); break; \
    default: HIF8_GDN_TOKEN(R, 4); break; \
  }
  if (rep == 2) HIF8_GDN_TOKEN_W(2)
  else HIF8_GDN_TOKEN_W(1)
#undef HIF8_GDN_TOKEN_W
#undef HIF8_GDN_TOKEN
  return check_launch("hif8_gdn_decode_token");
}

extern "C" int hif8_gdn_decode_head(const float *conv, const uint16_t *mixed_qkvz, int64_t ld, const uint16_t *x,
                                    const uint16_t *ba_weight, int64_t hidden, const float *a_log,
                                    const float *dt_bias, float *rec_state, const uint16_t *out_norm, uint16_t *out,
                                    int64_t batch, int64_t k_heads, int64_t v_heads, int64_t k_dim, int64_t v_dim,
                                    float eps, hif8_stream_t stream) {
  clear_error();
  if (!conv || !mixed_qkvz || !x || !ba_weight || !a_log || !dt_bias || !rec_state || !out_norm || !out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_head: null pointer argument");
  if (batch <= 0 || k_heads <= 0 || v_heads <= 0 || v_heads % k_heads || k_dim <= 0 || v_dim <= 0 ||
      hidden <= 0 || hidden > 0x7FFFFFFFll || batch * v_heads > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_head: unsupported dimensions");
  const int64_t channels = 2 * k_heads * k_dim + v_heads * v_dim;
  if (ld < channels + v_heads * v_dim)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_head: mixed_qkvz row too short");
  const int64_t rows = k_dim / kGdnParts;
  if (k_dim % kGdnParts || (rows != 16 && rows != 8 && rows != 4) || v_dim > kGdnCols || hidden % 8 ||
      hidden > 8 * kNormThreads * 4 || !aligned(x, 16) || !aligned(ba_weight, 16))
    return fail(HIF8_ERR_UNSUPPORTED, "hif8_gdn_decode_head: needs k_dim in {32, 64, 128}, v_dim <= 128, "
                                      "hidden %% 8 == 0, hidden <= 8192 and 16-byte aligned x / ba_weight");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(unsigned(batch * v_heads));
#define HIF8_GDN_HEAD(R)                                                                                    \
  gdn_head_kernel<R><<<grid, kGdnWideThreads, 0, s>>>(conv, mixed_qkvz, ld, x, ba_weight, int(hidden), a_log, \
                                                      dt_bias, rec_state, out_norm, out, int(k_heads),        \
                                                      int(v_heads), int(v_dim), eps)
  if (rows == 16) HIF8_GDN_HEAD(16);
  else if (rows == 8) HIF8_GDN_HEAD(8);
  else HIF8_GDN_HEAD(4);
#undef HIF8_GDN_HEAD
  return check_launch("hif8_gdn_decode_head");
}

extern "C" int hif8_gdn_decode_step(const uint16_t *mixed_qkvz, int64_t ld, const uint16_t *ba,
                                    const uint16_t *conv_weight, uint16_t *conv_state, const float *a_log,
                                    const float *dt_bias, float *rec_state, const uint16_t *out_norm,
                                    uint16_t *out, float *conv_scratch, int64_t batch, int64_t k_heads,
                                    int64_t v_heads, int64_t k_dim, int64_t v_dim, int64_t conv_width, float eps,
                                    hif8_stream_t stream) {
  clear_error();
  if (!mixed_qkvz || !ba || !conv_weight || !conv_state || !a_log || !dt_bias || !rec_state || !out_norm || !out ||
      !conv_scratch)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_step: null pointer argument");
  if (batch <= 0 || k_heads <= 0 || v_heads <= 0 || v_heads % k_heads || k_dim <= 0 || v_dim <= 0 ||
      k_dim > kGdnThreads || v_dim > kGdnThreads || conv_width < 2 || conv_width > 16 || batch > 65536)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_step: unsupported dimensions");
  const int64_t channels = 2 * k_heads * k_dim + v_heads * v_dim;
  if (ld < channels + v_heads * v_dim)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gdn_decode_step: mixed_qkvz row too short");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t items = batch * channels;
  gdn_conv_kernel<<<unsigned((items + 255) / 256), 256, 0, s>>>(mixed_qkvz, ld, int(channels), conv_weight,
                                                                conv_state, conv_scratch, int(batch),
                                                                int(conv_width));
  int st = check_launch("hif8_gdn_decode_step (conv)");
  if (st) return st;
  if (k_dim % kGdnParts == 0 && k_dim <= kGdnParts * kGdnRows && v_dim <= kGdnCols)
    gdn_delta_wide_kernel<<<unsigned(batch * v_heads), kGdnWideThreads, 0, s>>>(
        conv_scratch, int(channels), mixed_qkvz, ld, ba, a_log, dt_bias, rec_state, out_norm, out, int(k_heads),
        int(v_heads), int(k_dim), int(v_dim), eps);
  else
    gdn_delta_kernel<<<unsigned(batch * v_heads), kGdnThreads, 0, s>>>(
        conv_scratch, int(channels), mixed_qkvz, ld, ba, a_log, dt_bias, rec_state, out_norm, out, int(k_heads),
        int(v_heads), int(k_dim), int(v_dim), eps);
  return check_launch("hif8_gdn_decode_step (delta rule)");
}
