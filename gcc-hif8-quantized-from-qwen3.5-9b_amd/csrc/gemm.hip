// Prefill GEMM for gfx950: C[m, n] = sum_k dec(A[m,k]) dec(W[n,k]) * ts[m] * cs[n] (+ b[n]).
//
// Both operands are K-contiguous HiF8 bytes.  A block stages BM x 64 and
// BN x 64 byte tiles: each thread loads 16-byte chunks from global memory into
// VGPRs, decodes them with the 256-entry bf16 table in LDS and writes the bf16
// tile into LDS (double buffered, 16-byte granules XOR-swizzled by row so the
// MFMA fragment reads are bank-conflict free).  Four wavefronts in a 2 x 2
// arrangement each own a (BM/2) x (BN/2) sub-tile and run
// v_mfma_f32_16x16x32_bf16 with FP32 accumulation.  HiF8 values are exact in
// bf16, so the product is exact up to FP32 summation order.  The next k-step's
// global loads are in flight while the current step's MFMAs run.
// The epilogue applies acc * ts[m] * cs[n] (+ bias) and rounds once.
#include <stdlib.h>

#include "linear.h"

namespace hif8 {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 64;  // bytes (= bf16 elements) of K per stage
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// LDS byte offset of 16-byte granule g (0..7) of tile row r; rows are 128 bytes.
__device__ __forceinline__ uint32_t granule_offset(int r, int g) {
  return uint32_t(r) * 128u + uint32_t((g ^ (r & 7)) * 16);
}

__device__ __forceinline__ void decode16(const uint16_t *lut, const u32x4 q, u32x4 &lo, u32x4 &hi) {
  uint32_t p[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = q[i];
    p[2 * i] = uint32_t(lut[w & 0xFFu]) | (uint32_t(lut[(w >> 8) & 0xFFu]) << 16);
    p[2 * i + 1] = uint32_t(lut[(w >> 16) & 0xFFu]) | (uint32_t(lut[w >> 24]) << 16);
  }
  lo = u32x4{p[0], p[1], p[2], p[3]};
  hi = u32x4{p[4], p[5], p[6], p[7]};
}

// Static LDS table at address 0 (the only static LDS object of the kernel):
// a lookup address is then the code shifted left by one, a single SDWA op.
template <int kBM, int kBN, int kWavesM, int kWavesN>
__global__ __launch_bounds__(kWave * kWavesM * kWavesN, 1) void gemm_kernel(
    const uint8_t *__restrict__ A, const float *__restrict__ ts, const uint8_t *__restrict__ W,
    const float *__restrict__ cs, const void *__restrict__ bias, int bias_dtype,
    void *__restrict__ out, int out_dtype, int M, int N, int K) {
  constexpr int kT = kWave * kWavesM * kWavesN;         // threads per block
  constexpr int kChunksA = kBM * (kBK / 16) / kT;        // 16-byte chunks per thread
  constexpr int kChunksB = kBN * (kBK / 16) / kT;
  constexpr int kRowsPass = kT / 4;                      // tile rows covered per chunk pass
  constexpr int kWM = kBM / kWavesM, kWN = kBN / kWavesN;  // wave sub-tile
  constexpr int kTM = kWM / 16, kTN = kWN / 16;          // 16x16 MFMA tiles per wave
  constexpr uint32_t kStageA = kBM * kBK * 2, kStageB = kBN * kBK * 2;
  constexpr int kGroupM = 4;                             // row tiles per L2 group

  __shared__ __attribute__((aligned(16))) uint16_t lut[256];
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t *sa = smem;
  uint8_t *sb = sa + 2 * kStageA;

  const int tid = threadIdx.x;
  if (tid < 256) lut[tid] = kDeviceTables.decode_bf16[tid];

  // Tile order: the blocks of one XCD (block id modulo 8) take a contiguous
  // range of tiles, walked in groups of kGroupM row tiles so that blocks
  // running together share A row panels and B column panels in that XCD's L2.
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  const int tiles = tiles_m * tiles_n;
  const int per_xcd = (tiles + 7) / 8;
  const int lin = (int(blockIdx.x) & 7) * per_xcd + (int(blockIdx.x) >> 3);
  if (lin >= tiles) return;
  const int group = lin / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int group_rows = min(tiles_m - first_m, kGroupM);
  const int in_group = lin - group * kGroupM * tiles_n;
  const int m0 = (first_m + in_group % group_rows) * kBM;
  const int n0 = (in_group / group_rows) * kBN;

  const int wave = tid / kWave, lane = tid % kWave;
  const int wm = wave / kWavesN, wn = wave % kWavesN;

  // Global chunk coordinates: 4 threads per 64-byte tile row.
  const int crow = tid >> 2, ccol = tid & 3;
  const uint8_t *pa[kChunksA];
  const uint8_t *pb[kChunksB];
#pragma unroll
  for (int i = 0; i < kChunksA; ++i) {
    const int r = min(m0 + crow + kRowsPass * i, M - 1);
    pa[i] = A + size_t(r) * K + ccol * 16;
  }
#pragma unroll
  for (int i = 0; i < kChunksB; ++i) {
    const int r = min(n0 + crow + kRowsPass * i, N - 1);
    pb[i] = W + size_t(r) * K + ccol * 16;
  }

  u32x4 ra[kChunksA], rb[kChunksB];
  auto load = [&](int kt) {
#pragma unroll
    for (int i = 0; i < kChunksA; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(pa[i] + kt * kBK);
#pragma unroll
    for (int i = 0; i < kChunksB; ++i) rb[i] = *reinterpret_cast<const u32x4 *>(pb[i] + kt * kBK);
  };
  // Decode one 16-byte chunk and store its two bf16 granules.
  auto put = [&](uint8_t *d, int r, const u32x4 q) {
    u32x4 lo, hi;
    decode16(lut, q, lo, hi);
    *reinterpret_cast<u32x4 *>(d + granule_offset(r, 2 * ccol)) = lo;
    *reinterpret_cast<u32x4 *>(d + granule_offset(r, 2 * ccol + 1)) = hi;
  };
  auto store = [&](int stage) {
#pragma unroll
    for (int i = 0; i < kChunksA; ++i) put(sa + stage * kStageA, crow + kRowsPass * i, ra[i]);
#pragma unroll
    for (int i = 0; i < kChunksB; ++i) put(sb + stage * kStageB, crow + kRowsPass * i, rb[i]);
  };

  f32x4_t acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int KT = K / kBK;
  load(0);
  __syncthreads();  // lut ready
  store(0);
  if (KT > 1) load(1);
  __syncthreads();

  const int frow = lane & 15, fgrp = lane >> 4;
  for (int kt = 0; kt < KT; ++kt) {
    const int stage = kt & 1;
    const uint8_t *da = sa + stage * kStageA;
    const uint8_t *db = sb + stage * kStageB;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8_t af[kTM], bfr[kTN];
#pragma unroll
      for (int i = 0; i < kTM; ++i) {
        const int r = wm * kWM + i * 16 + frow;
        af[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4 *>(da + granule_offset(r, kk * 4 + fgrp)));
      }
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        const int r = wn * kWN + j * 16 + frow;
        bfr[j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4 *>(db + granule_offset(r, kk * 4 + fgrp)));
      }
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    // The next tile (loaded during the previous step) goes to the other
    // stage while this step's MFMAs drain; then the tile after it is loaded.
    if (kt + 1 < KT) {
      store(stage ^ 1);
      if (kt + 2 < KT) load(kt + 2);
    }
    __syncthreads();
  }

  // Epilogue: D[i][j] of a 16x16 tile lives in lane (i/4)*16 + j, element i%4.
  uint16_t *o = static_cast<uint16_t *>(out);
  const bool obf = out_dtype == HIF8_DTYPE_BF16;
  float rs[kTM][4];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) rs[i][e] = ts[min(m0 + wm * kWM + i * 16 + fgrp * 4 + e, M - 1)];
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const int col = n0 + wn * kWN + j * 16 + frow;
    if (col >= N) continue;
    const float c = cs[col];
    float b = 0.f;
    if (bias) {
      const uint16_t h = static_cast<const uint16_t *>(bias)[col];
      b = bias_dtype == HIF8_DTYPE_BF16 ? half_bits_to_float<true>(h) : half_bits_to_float<false>(h);
    }
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wm * kWM + i * 16 + fgrp * 4 + e;
        if (row < M) {
          const float y = acc[i][j][e] * rs[i][e] * c + b;
          o[size_t(row) * N + col] = obf ? float_to_bf16_bits(y) : float_to_f16_bits(y);
        }
      }
    }
  }
}

// Any shape: one thread per output element.
__global__ __launch_bounds__(256) void gemm_simple_kernel(
    const uint8_t *__restrict__ A, const float *__restrict__ ts, const uint8_t *__restrict__ W,
    const float *__restrict__ cs, const void *__restrict__ bias, int bias_dtype,
    void *__restrict__ out, int out_dtype, int M, int N, int K) {
  const int col = blockIdx.x * 256 + threadIdx.x;
  const int row = blockIdx.y;
  if (col >= N) return;
  const uint8_t *a = A + size_t(row) * K;
  const uint8_t *w = W + size_t(col) * K;
  float acc = 0.f;
  for (int kk = 0; kk < K; ++kk)
    acc = fmaf(__uint_as_float(kDeviceTables.decode_f32[a[kk]]),
               __uint_as_float(kDeviceTables.decode_f32[w[kk]]), acc);
  float y = acc * ts[row] * cs[col];
  if (bias) {
    const uint16_t h = static_cast<const uint16_t *>(bias)[col];
    y += bias_dtype == HIF8_DTYPE_BF16 ? half_bits_to_float<true>(h) : half_bits_to_float<false>(h);
  }
  static_cast<uint16_t *>(out)[size_t(row) * N + col] =
      out_dtype == HIF8_DTYPE_BF16 ? float_to_bf16_bits(y) : float_to_f16_bits(y);
}

template <int kBM, int kBN, int kWavesM, int kWavesN>
int launch_tiled(const LinearArgs &a) {
  constexpr size_t kSmem = 2 * size_t(kBM + kBN) * kBK * 2;  // + 512 B of static LDS (the table)
  constexpr int kT = kWave * kWavesM * kWavesN;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_kernel<kBM, kBN, kWavesM, kWavesN>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(kSmem)) != hipSuccess)
      return fail(HIF8_ERR_LAUNCH, "soft_hif8 GEMM: cannot reserve %zu bytes of LDS", kSmem);
    configured = true;
  }
  const int64_t tiles = ((a.n + kBN - 1) / kBN) * ((a.m + kBM - 1) / kBM);
  const dim3 grid(unsigned((tiles + 7) / 8 * 8));
  gemm_kernel<kBM, kBN, kWavesM, kWavesN><<<grid, kT, kSmem, a.stream>>>(
      static_cast<const uint8_t *>(a.act), a.act_scale, a.weight, a.channel_scale, a.bias,
      a.bias_dtype, a.out, a.out_dtype, int(a.m), int(a.n), int(a.k));
  return check_launch("soft_hif8 GEMM");
}

}  // namespace

int launch_gemm(const LinearArgs &a) {
  if (a.act_kind != kActCodes)
    return fail(HIF8_ERR_UNSUPPORTED, "soft_hif8 GEMM takes uint8 activation codes");
  const bool tiled = a.k % kBK == 0 && aligned(a.act, 16) && aligned(a.weight, 16);
  if (!tiled) {
    const dim3 grid(unsigned((a.n + 255) / 256), unsigned(a.m));
    gemm_simple_kernel<<<grid, 256, 0, a.stream>>>(
        static_cast<const uint8_t *>(a.act), a.act_scale, a.weight, a.channel_scale, a.bias,
        a.bias_dtype, a.out, a.out_dtype, int(a.m), int(a.n), int(a.k));
    return check_launch("soft_hif8 GEMM (generic)");
  }
  const int64_t tiles256 = ((a.m + 255) / 256) * ((a.n + 255) / 256);
  static const int variant = getenv("HIF8_GEMM_WAVES") ? atoi(getenv("HIF8_GEMM_WAVES")) : 8;
  if (a.m >= 256 && tiles256 >= 128) {
    if (variant == 4) return launch_tiled<256, 256, 2, 2>(a);
    return launch_tiled<256, 256, 2, 4>(a);
  }
  return launch_tiled<128, 128, 2, 2>(a);
}

}  // namespace hif8
