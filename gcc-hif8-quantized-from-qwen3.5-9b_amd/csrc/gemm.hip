// Prefill GEMM for gfx950: C[m, n] = sum_k dec(A[m,k]) dec(W[n,k]) * ts[m] * cs[n] (+ b[n]).
//
// Both operands are K-contiguous HiF8 bytes.  HiF8 values are exact in bf16,
// so the operands are decoded to bf16 and multiplied on
// v_mfma_f32_16x16x32_bf16 with FP32 accumulation: the product is exact up to
// FP32 summation order.  The epilogue applies acc * ts[m] * cs[n] (+ bias) and
// rounds once.
//
// A block computes a BM x BN tile in K steps of 64.  Each step's tiles sit in
// LDS as bf16 (double buffered, 16-byte granules XOR-swizzled by row so that
// the MFMA fragment reads are bank-conflict free).  Two kernels:
//   * gemm_kernel, W decoded in the kernel: each thread loads 16-byte W code
//     chunks into VGPRs one step ahead, decodes them with the 256-entry bf16
//     table in LDS and stores the bf16 granules.  With a workspace the
//     activation codes are first decoded once to a bf16 matrix
//     (decode_rows_kernel) and every step copies its A tile straight into
//     LDS with global_load_lds_dwordx4; without one A is decoded like W.
//     256 x 256 blocks run eight wavefronts in a 2 x 4 arrangement (128 x 64
//     each, two waves per SIMD) whose two wave rows alternate between MFMA
//     and decode half a step apart; 128 x 128 blocks run four in 2 x 2.
//   * gemm_dma_kernel, both operands bf16 in HBM: the weight decoded once per
//     call (M >= 2048, where the in-kernel decode would repeat per 256-row
//     tile of M) or kept decoded by the caller (soft_hif8_gemm_decoded_weight).
//     Every step copies both tiles into LDS by DMA and the K loop is MFMAs
//     and fragment reads in a hand-pinned order (4 x 2 waves of 64 x 128).
// The epilogue scales and rounds each wave's outputs into LDS and stores
// them as 16-byte row chunks (full 128-byte row segments per 8 lanes).
//
// Shapes with too few output tiles to fill 256 CUs (prefill M=512, narrow N)
// split K: block (tile, s) sums K steps [s*ksteps, (s+1)*ksteps) and stores
// its FP32 tile to partial[s][M][N]; a second kernel adds the splits in fixed
// order and applies the same epilogue, so results are deterministic.
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "linear.h"

namespace hif8 {
namespace {

constexpr int kBK = 64;  // bytes (= bf16 elements) of K per stage
constexpr int kMaxDmaK = 1 << 23;  // gemm_dma_kernel: a tile's rows in 32-bit byte offsets
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// LDS byte offset of 16-byte granule g (0..7) of tile row r; rows are 128 bytes.
__device__ __forceinline__ uint32_t granule_offset(int r, int g) {
  return uint32_t(r) * 128u + uint32_t((g ^ (r & 7)) * 16);
}

// 16 codes -> 16 bf16 (lo = codes 0..7, hi = codes 8..15) via the LDS table.
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

// Codes [rows, K] -> bf16 [rows, K], 16 codes per thread and pass, over one
// or two independent ranges (a: `chunks` 16-code chunks into out, then b:
// `chunks_b` chunks into out_b), walked as one index space so that one launch
// decodes both GEMM operands.  The table is computed (one entry per thread),
// so the first chunk's load goes out before it and stays in flight across the
// LDS-only barrier; each pass loads the next chunk before decoding the
// current one (a chunk past the end re-reads the last one, unused).
__global__ __launch_bounds__(256) void decode_rows_kernel(const uint8_t *__restrict__ a,
                                                          uint16_t *__restrict__ out, size_t chunks,
                                                          const uint8_t *__restrict__ b,
                                                          uint16_t *__restrict__ out_b, size_t chunks_b) {
  __shared__ __attribute__((aligned(16))) uint16_t lut[256];
  const size_t total = chunks + chunks_b;
  if (total == 0) return;
  const size_t stride = size_t(gridDim.x) * 256;
  size_t c = size_t(blockIdx.x) * 256 + threadIdx.x;
  auto fetch = [&](size_t ch) {
    ch = ch < total ? ch : total - 1;
    return *reinterpret_cast<const u32x4 *>(ch < chunks ? a + ch * 16 : b + (ch - chunks) * 16);
  };
  u32x4 q = fetch(c);
  lut[threadIdx.x] = uint16_t(decode_bits(threadIdx.x) >> 16);
  lds_barrier();
  for (; c < total; c += stride) {
    const u32x4 cur = q;
    q = fetch(c + stride);
    u32x4 lo, hi;
    decode16(lut, cur, lo, hi);
    u32x4 *o = reinterpret_cast<u32x4 *>(c < chunks ? out + c * 16 : out_b + (c - chunks) * 16);
    o[0] = lo;
    o[1] = hi;
  }
}

// Tile order: the blocks of one XCD (block id modulo 8) take a contiguous
// range of tiles, walked in groups of 4 row tiles so that blocks running
// together share A row panels and B column panels in that XCD's L2.  The K
// splits of a tile are adjacent work units, so they run on one XCD.  Returns
// false for the padding blocks of the grid.
template <int kBM, int kBN>
__device__ __forceinline__ bool tile_of(int M, int N, int splits, int &m0, int &n0, int &split) {
  constexpr int kGroupM = 4;
  const int tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  const int units = tiles_m * tiles_n * splits;
  const int per_xcd = (units + 7) / 8;
  const int unit = (int(blockIdx.x) & 7) * per_xcd + (int(blockIdx.x) >> 3);
  if (unit >= units) return false;
  const int lin = unit / splits;
  split = unit - lin * splits;
  const int group = lin / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int group_rows = min(tiles_m - first_m, kGroupM);
  const int in_group = lin - group * kGroupM * tiles_n;
  m0 = (first_m + in_group % group_rows) * kBM;
  n0 = (in_group / group_rows) * kBN;
  return true;
}

// Epilogue of a wave's kTM x kTN grid of 16x16 MFMA tiles whose top-left
// output is (r0, c0).  D[i][j] of a 16x16 tile lives in lane (i/4)*16 + j,
// element i%4.  With split-K partials the raw FP32 sums go to
// partial[split][M][N]; otherwise out = acc * ts[row] * cs[col] (+ bias),
// rounded once.
template <int kTM, int kTN>
__device__ __forceinline__ void store_tile(const f32x4_t (&acc)[kTM][kTN], int r0, int c0, int frow, int fgrp,
                                           const float *__restrict__ ts, const float *__restrict__ cs,
                                           const void *__restrict__ bias, int bias_dtype,
                                           void *__restrict__ out, int out_dtype, int M, int N,
                                           float *__restrict__ partial, int split) {
  if (partial) {
    float *p = partial + size_t(split) * M * N;
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int col = c0 + j * 16 + frow;
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = r0 + i * 16 + fgrp * 4 + e;
          if (row < M) p[size_t(row) * N + col] = acc[i][j][e];
        }
    }
    return;
  }
  uint16_t *o = static_cast<uint16_t *>(out);
  const bool obf = out_dtype == HIF8_DTYPE_BF16;
  float rs[kTM][4];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) rs[i][e] = ts[min(r0 + i * 16 + fgrp * 4 + e, M - 1)];
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const int col = c0 + j * 16 + frow;
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
        const int row = r0 + i * 16 + fgrp * 4 + e;
        if (row < M) {
          const float y = acc[i][j][e] * rs[i][e] * c + b;
          o[size_t(row) * N + col] = obf ? float_to_bf16_bits(y) : float_to_f16_bits(y);
        }
      }
    }
  }
}

// Epilogue through LDS for 16-bit outputs: the wave's outputs, scaled and
// rounded, go to its own LDS region (row pitch kWN * 2 + 16 bytes, so the
// four 4-row groups of a 16x16 tile fall in different banks) and come back
// as 16-byte row chunks, each stored with one 16-byte store: 8 lanes write a
// 128-byte row segment instead of 16 lanes writing 32 bytes with 2-byte
// stores.  The caller has retired every read of the LDS stages.
template <int kTM, int kTN>
constexpr int epilogue_region_bytes() {
  return kTM * 16 * (kTN * 16 * 2 + 16);
}

template <int kTM, int kTN>
__device__ __forceinline__ void store_tile_lds(const f32x4_t (&acc)[kTM][kTN], uint8_t *region, int r0, int c0,
                                               int lane, const float *__restrict__ ts, const float *__restrict__ cs,
                                               const void *__restrict__ bias, int bias_dtype,
                                               void *__restrict__ out, int out_dtype, int M, int N) {
  constexpr int kWM = kTM * 16, kWN = kTN * 16, kPitch = kWN * 2 + 16;
  const int frow = lane & 15, fgrp = lane >> 4;
  const bool obf = out_dtype == HIF8_DTYPE_BF16;
  float rs[kTM][4];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) rs[i][e] = ts[min(r0 + i * 16 + fgrp * 4 + e, M - 1)];
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const int cl = j * 16 + frow;
    const int col = min(c0 + cl, N - 1);
    const float c = cs[col];
    float b = 0.f;
    if (bias) {
      const uint16_t h = static_cast<const uint16_t *>(bias)[col];
      b = bias_dtype == HIF8_DTYPE_BF16 ? half_bits_to_float<true>(h) : half_bits_to_float<false>(h);
    }
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y = acc[i][j][e] * rs[i][e] * c + b;
        *reinterpret_cast<uint16_t *>(region + (i * 16 + fgrp * 4 + e) * kPitch + cl * 2) =
            obf ? float_to_bf16_bits(y) : float_to_f16_bits(y);
      }
  }
  // LDS operations of one wave complete in order; the wait and the fences
  // keep the compiler from moving the reads above the writes.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_wave_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  constexpr int kRowChunks = kWN / 8;
  constexpr int kPerLane = kWM * kRowChunks / kWave;
  uint16_t *o = static_cast<uint16_t *>(out);
  const bool vec = (N % 8 == 0) && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
#pragma unroll
  for (int t = 0; t < kPerLane; ++t) {
    const int ch = lane + kWave * t;
    const int rl = ch / kRowChunks, cc = (ch % kRowChunks) * 8;
    const u32x4 v = *reinterpret_cast<const u32x4 *>(region + rl * kPitch + cc * 2);
    const int row = r0 + rl, col = c0 + cc;
    if (row >= M || col >= N) continue;
    uint16_t *dst = o + size_t(row) * N + col;
    if (vec && col + 8 <= N) {
      *reinterpret_cast<u32x4 *>(dst) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (col + e < N) dst[e] = uint16_t(v[e >> 1] >> ((e & 1) * 16));
    }
  }
}

// Static LDS table at address 0 (the only static LDS object of the kernel):
// a lookup address is then the code shifted left by one, a single SDWA op.
//   kAPre      A is a bf16 matrix (decoded beforehand) copied into LDS by DMA
//   kPingPong  the two wave rows alternate MFMA and decode half a step apart
template <int kBM, int kBN, int kWavesM, int kWavesN, bool kAPre, bool kPingPong>
__global__ __launch_bounds__(kWave * kWavesM * kWavesN, 1) void gemm_kernel(
    const void *__restrict__ A, const float *__restrict__ ts, const void *__restrict__ W,
    const float *__restrict__ cs, const void *__restrict__ bias, int bias_dtype,
    void *__restrict__ out, int out_dtype, int M, int N, int K, float *__restrict__ partial,
    int splits, int ksteps) {
  constexpr int kT = kWave * kWavesM * kWavesN;         // threads per block
  constexpr int kWaves = kWavesM * kWavesN;
  static_assert(!kPingPong || kWavesM == 2, "ping-pong pairs the two wave rows");
  // Threads sharing one decode: all of them, or (ping-pong) one wave row,
  // which decodes its half of the A rows and its half of the W rows.
  constexpr int kDecT = kPingPong ? kT / 2 : kT;
  constexpr int kDecA = kPingPong ? kBM / 2 : kBM, kDecB = kPingPong ? kBN / 2 : kBN;
  constexpr int kChunksA = kAPre ? 0 : kDecA * (kBK / 16) / kDecT;  // 16-byte code chunks per thread
  constexpr int kChunksB = kDecB * (kBK / 16) / kDecT;
  constexpr int kRowsPass = kDecT / 4;                   // tile rows covered per chunk pass
  constexpr int kWM = kBM / kWavesM, kWN = kBN / kWavesN;  // wave sub-tile
  constexpr int kTM = kWM / 16, kTN = kWN / 16;          // 16x16 MFMA tiles per wave
  constexpr uint32_t kStageA = kBM * kBK * 2, kStageB = kBN * kBK * 2;
  // Tiles by DMA: 1 KiB (8 rows) per instruction, spread over the waves.
  constexpr int kDmaPerWave = kBM * kBK * 2 / 1024 / kWaves;
  static_assert(!kAPre || kDmaPerWave * kWaves * 1024 == int(kStageA), "A tile DMA split");

  __shared__ __attribute__((aligned(16))) uint16_t lut[256];
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t *sa = smem;
  uint8_t *sb = sa + 2 * kStageA;

  const int tid = threadIdx.x;
  if (tid < 256) lut[tid] = kDeviceTables.decode_bf16[tid];

  int m0, n0, split;
  if (!tile_of<kBM, kBN>(M, N, splits, m0, n0, split)) return;
  const size_t k_first = size_t(split) * ksteps * kBK;

  const int wave = tid / kWave, lane = tid % kWave;
  const int wm = wave / kWavesN, wn = wave % kWavesN;

  // Global chunk coordinates: 4 threads per 64-byte tile row.
  const int dt = tid % kDecT, crow = dt >> 2, ccol = dt & 3;
  const int base_a = kPingPong ? wm * kDecA : 0, base_b = kPingPong ? wm * kDecB : 0;
  const uint8_t *pa[kChunksA > 0 ? kChunksA : 1];
  const uint8_t *pb[kChunksB > 0 ? kChunksB : 1];
  if constexpr (kChunksA > 0) {
#pragma unroll
    for (int i = 0; i < kChunksA; ++i) {
      const int r = min(m0 + base_a + crow + kRowsPass * i, M - 1);
      pa[i] = static_cast<const uint8_t *>(A) + size_t(r) * K + k_first + ccol * 16;
    }
  }
  if constexpr (kChunksB > 0) {
#pragma unroll
    for (int i = 0; i < kChunksB; ++i) {
      const int r = min(n0 + base_b + crow + kRowsPass * i, N - 1);
      pb[i] = static_cast<const uint8_t *>(W) + size_t(r) * K + k_first + ccol * 16;
    }
  }

  // DMA source of this lane for the A tile (bf16 rows of 128 bytes per step):
  // instruction j of this wave fills LDS bytes [1024 q, 1024 q + 1024),
  // q = wave * kDmaPerWave + j, i.e. tile rows 8q..8q+7; lane i lands at
  // 1024 q + 16 i = row 8q + i/8, swizzled slot i%8, which holds granule
  // (i%8) ^ (row & 7).
  const uint8_t *pdma[kAPre ? kDmaPerWave : 1];
  if constexpr (kAPre) {
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int q = wave * kDmaPerWave + j;
      const int r = 8 * q + (lane >> 3);
      const int g = (lane & 7) ^ (r & 7);
      pdma[j] = static_cast<const uint8_t *>(A) + (size_t(min(m0 + r, M - 1)) * K + k_first + g * 8) * 2;
    }
  }
  auto dma_a = [&](int kt, int stage) {
    if constexpr (kAPre) {
      const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_address(sa + stage * kStageA)) +
                           uint32_t(wave * kDmaPerWave) * 1024u;
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) dma16(pdma[j] + size_t(kt) * kBK * 2, dst + 1024u * j);
    }
  };

  u32x4 ra[kChunksA > 0 ? kChunksA : 1], rb[kChunksB > 0 ? kChunksB : 1];
  auto load = [&](int kt) {
    if constexpr (kChunksA > 0) {
#pragma unroll
      for (int i = 0; i < kChunksA; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(pa[i] + kt * kBK);
    }
    if constexpr (kChunksB > 0) {
#pragma unroll
      for (int i = 0; i < kChunksB; ++i) rb[i] = *reinterpret_cast<const u32x4 *>(pb[i] + kt * kBK);
    }
  };
  // Decode one 16-byte chunk and store its two bf16 granules.
  auto put = [&](uint8_t *d, int r, const u32x4 q) {
    u32x4 lo, hi;
    decode16(lut, q, lo, hi);
    *reinterpret_cast<u32x4 *>(d + granule_offset(r, 2 * ccol)) = lo;
    *reinterpret_cast<u32x4 *>(d + granule_offset(r, 2 * ccol + 1)) = hi;
  };
  auto store = [&](int stage) {
    if constexpr (kChunksA > 0) {
#pragma unroll
      for (int i = 0; i < kChunksA; ++i) put(sa + stage * kStageA, base_a + crow + kRowsPass * i, ra[i]);
    }
    if constexpr (kChunksB > 0) {
#pragma unroll
      for (int i = 0; i < kChunksB; ++i) put(sb + stage * kStageB, base_b + crow + kRowsPass * i, rb[i]);
    }
  };

  f32x4_t acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int frow = lane & 15, fgrp = lane >> 4;
  auto compute = [&](int stage) {
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
  };

  // Prologue: tile 0 in stage 0, tile 1's codes in registers.  With the DMA
  // path the only loads in flight after the A copy are this thread's kChunksB
  // code loads, so waiting for vmcnt <= kChunksB retires the copy.
  const int KT = ksteps;
  dma_a(0, 0);
  load(0);
  __syncthreads();  // table ready
  store(0);
  load(min(1, KT - 1));
  if constexpr (kAPre) wait_vmcnt<kChunksB>();
  __syncthreads();

  if constexpr (kPingPong) {
    // The two wave rows alternate between MFMA and decode half a step apart:
    // while row 0 multiplies tile kt, row 1 decodes its half of tile kt+1;
    // then row 1 multiplies tile kt while row 0 decodes its half.  Each SIMD
    // holds one wave of each row, so the MFMA pipe is fed while the other
    // wave decodes.  Tile kt+1 is complete (both halves) before either row
    // multiplies it, and a stage is rewritten only after both rows read it.
    // The A copy of tile kt+1 is issued by every wave at the top of step kt.
    const bool second = wm == 1;
    for (int kt = 0; kt < KT; ++kt) {
      const int stage = kt & 1;
      const bool more = kt + 1 < KT;
      if (more) dma_a(kt + 1, stage ^ 1);
      if (!second) {
        __builtin_amdgcn_s_setprio(1);
        compute(stage);
        __builtin_amdgcn_s_setprio(0);
      } else if (more) {
        store(stage ^ 1);
        load(min(kt + 2, KT - 1));
      }
      lds_barrier();
      if (second) {
        __builtin_amdgcn_s_setprio(1);
        compute(stage);
        __builtin_amdgcn_s_setprio(0);
      } else if (more) {
        store(stage ^ 1);
        load(min(kt + 2, KT - 1));
      }
      if constexpr (kAPre) wait_vmcnt<kChunksB>();
      lds_barrier();
    }
  } else {
    // All waves: start the A copy of the next tile, the MFMAs of this stage,
    // then the decode of the W codes loaded during the previous step into
    // the other stage and the loads of the tile after it (the last one is
    // loaded again rather than branched around).  The barrier waits for LDS
    // traffic only; the copy is retired by the vmcnt wait before it.
    for (int kt = 0; kt + 1 < KT; ++kt) {
      dma_a(kt + 1, (kt & 1) ^ 1);
      compute(kt & 1);
      store((kt & 1) ^ 1);
      load(min(kt + 2, KT - 1));
      if constexpr (kAPre) wait_vmcnt<kChunksB>();
      lds_barrier();
    }
    compute((KT - 1) & 1);
  }
  // No copy may still target LDS when the wave ends (the last load() above
  // only re-reads the final tile into registers).
  if constexpr (kAPre) wait_vmcnt<0>();

  if (partial) {
    store_tile<kTM, kTN>(acc, m0 + wm * kWM, n0 + wn * kWN, frow, fgrp, ts, cs, bias, bias_dtype, out, out_dtype,
                         M, N, partial, split);
    return;
  }
  lds_barrier();  // every wave is done reading the stages
  store_tile_lds<kTM, kTN>(acc, smem + wave * epilogue_region_bytes<kTM, kTN>(), m0 + wm * kWM, n0 + wn * kWN, lane,
                           ts, cs, bias, bias_dtype, out, out_dtype, M, N);
}

// Both operands already bf16 (A decoded once per call, W decoded once per
// call or kept decoded by the caller): every K step copies the A and W tiles
// into LDS by DMA and the K loop is MFMAs and fragment reads only, scheduled
// by hand.  A K step of 64 is two 32-wide slices; each wave holds the
// fragments of two slices in registers and reads the next slice's fragments
// while the MFMAs of the current one run (one ds_read_b128 between every few
// MFMAs: left to itself the compiler reads each fragment right before its
// first MFMA and waits for it there).  One barrier per step, between the two
// slices: after it the step's stage may be overwritten (the copy of step
// kt + 2 is issued right there) and the next step's tile has landed, so the
// second slice's MFMAs run while the next step's first fragments are read.
// Wave sub-tiles are kBM / kWavesM rows x kBN / kWavesN columns: each A
// fragment feeds kTN MFMAs in a row.
//
// kWDec: W is the uint8 code matrix, decoded in the kernel.  Each thread
// loads 16-byte code chunks of the W tile a step ahead into VGPRs; during the
// first slice of step kt it looks the codes of tile kt + 1 up in the 256-entry
// bf16 table (LDS address 0) and stores them into that tile's stage (free
// since the barrier of step kt - 1), lookups and the packing of their results
// a few MFMAs apart, then loads the codes of tile kt + 2.  The A tile still
// comes by DMA.
template <int kBM, int kBN, int kWavesM, int kWavesN, bool kWDec>
__global__ __launch_bounds__(kWave * kWavesM * kWavesN, 1) void gemm_dma_kernel(
    const uint16_t *__restrict__ A, const float *__restrict__ ts, const void *__restrict__ Wv,
    const float *__restrict__ cs, const void *__restrict__ bias, int bias_dtype,
    void *__restrict__ out, int out_dtype, int M, int N, int K, float *__restrict__ partial,
    int splits, int ksteps) {
  constexpr int kWaves = kWavesM * kWavesN;
  constexpr int kT = kWave * kWaves;
  constexpr int kWM = kBM / kWavesM, kWN = kBN / kWavesN;
  constexpr int kTM = kWM / 16, kTN = kWN / 16;
  constexpr uint32_t kStageA = kBM * kBK * 2, kStageB = kBN * kBK * 2, kStage = kStageA + kStageB;
  constexpr int kDmaA = int(kStageA) / 1024 / kWaves, kDmaB = kWDec ? 0 : int(kStageB) / 1024 / kWaves;
  static_assert(kDmaA * kWaves * 1024 == int(kStageA) && (kWDec || kDmaB * kWaves * 1024 == int(kStageB)),
                "tile copies split evenly over the waves");
  constexpr int kDec = kWDec ? kBN * kBK / 8 / kT : 0;  // 8-code W chunks per thread and step
  static_assert(!kWDec || kDec * 8 * kT == kBN * kBK, "W decode split evenly over the threads");
  const uint16_t *W = static_cast<const uint16_t *>(Wv);
  const uint8_t *Wc = static_cast<const uint8_t *>(Wv);
  constexpr int kReads = kTM + kTN, kMfmas = kTM * kTN;
  // MFMAs between two reads: the reads fill the first three quarters of a
  // slice, so the last one has a quarter of the slice to land.
  constexpr int kPerRead = kMfmas * 3 / 4 / kReads > 0 ? kMfmas * 3 / 4 / kReads : 1;

  // The decode table first (the only static LDS object: address 0), then the stages.
  __shared__ __attribute__((aligned(16))) uint16_t lut[kWDec ? 256 : 8];
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  int m0, n0, split;
  if (!tile_of<kBM, kBN>(M, N, splits, m0, n0, split)) return;
  const size_t k_first = size_t(split) * ksteps * kBK;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  if constexpr (kWDec) {
    if (tid < 256) lut[tid] = uint16_t(decode_bits(uint32_t(tid)) >> 16);
  }
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int frow = lane & 15, fgrp = lane >> 4;

  // Copy sources: instruction j of this wave fills 1 KiB q = wave * kDma + j
  // of the tile (rows 8q .. 8q + 7, 128 bytes each); lane i lands at row
  // 8q + i / 8, slot i % 8, which holds granule (i % 8) ^ (row & 7).  Byte
  // offsets from the tile's first row in this split (rows past the last one
  // read the last row); the host keeps kBM x K x 2 below 2^32.
  uint32_t oa[kDmaA], ob[kDmaB > 0 ? kDmaB : 1];
#pragma unroll
  for (int j = 0; j < kDmaA; ++j) {
    const int r = 8 * (wave * kDmaA + j) + (lane >> 3);
    oa[j] = uint32_t(min(m0 + r, M - 1) - m0) * uint32_t(K) * 2u + uint32_t((lane & 7) ^ (r & 7)) * 16u;
  }
#pragma unroll
  for (int j = 0; j < kDmaB; ++j) {
    const int r = 8 * (wave * kDmaB + j) + (lane >> 3);
    ob[j] = uint32_t(min(n0 + r, N - 1) - n0) * uint32_t(K) * 2u + uint32_t((lane & 7) ^ (r & 7)) * 16u;
  }
  const uint16_t *a_split = A + size_t(m0) * K + k_first, *w_split = W + size_t(n0) * K + k_first;
  const uint32_t lds0 = lds_address(smem);

  // W codes (kWDec): chunk c of this thread is q = tid + c * kT of the tile,
  // row q / 8, codes 8 (q % 8) .. 8 (q % 8) + 7 of the step's 64, which
  // decode to granule q % 8 of the row.
  uint32_t wco[kDec > 0 ? kDec : 1], wdst[kDec > 0 ? kDec : 1];
  uint2 wq[kDec > 0 ? kDec : 1];
  if constexpr (kWDec) {
#pragma unroll
    for (int c = 0; c < kDec; ++c) {
      const int q = tid + c * kT, r = q >> 3, gq = q & 7;
      wco[c] = uint32_t(min(n0 + r, N - 1) - n0) * uint32_t(K) + uint32_t(gq) * 8u;
      wdst[c] = kStageA + uint32_t(r) * 128u + uint32_t((gq ^ (r & 7)) * 16);
    }
  }
  const uint8_t *wc_split = Wc + size_t(n0) * K + k_first;
  auto load_codes = [&](int kt) {
#pragma unroll
    for (int c = 0; c < kDec; ++c) wq[c] = *reinterpret_cast<const uint2 *>(wc_split + size_t(kt) * kBK + wco[c]);
  };
  // Chunk c: looks up its 8 codes (8 table entries), then packs them into
  // its bf16 granule in the stage at `stage`.
  uint32_t lk[8];
  auto lookup = [&](int c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) lk[j] = lut[(((j >> 2) ? wq[c].y : wq[c].x) >> (8 * (j & 3))) & 0xFFu];
  };
  auto pack_store = [&](int c, uint8_t *stage) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = lk[2 * i] | (lk[2 * i + 1] << 16);
    *reinterpret_cast<u32x4 *>(stage + wdst[c]) = v;
  };
  auto copy = [&](int kt, int stage) {
    const uint32_t dst = __builtin_amdgcn_readfirstlane(lds0 + uint32_t(stage) * kStage);
    const uint16_t *sa = a_split + size_t(kt) * kBK, *sw = w_split + size_t(kt) * kBK;
#pragma unroll
    for (int j = 0; j < kDmaA; ++j) dma16_offset(sa, oa[j], dst + uint32_t(wave * kDmaA + j) * 1024u);
#pragma unroll
    for (int j = 0; j < kDmaB; ++j) dma16_offset(sw, ob[j], dst + kStageA + uint32_t(wave * kDmaB + j) * 1024u);
  };

  // Fragment of 16x16x32 tile (i, j), slice kk: lane holds row frow, K
  // elements 8 fgrp .. 8 fgrp + 7 of the slice, i.e. granule 4 kk + fgrp.
  // Rows of one fragment start at a multiple of 16, so the swizzle term is
  // frow & 7 for every fragment of the lane.
  const uint32_t g0 = uint32_t((fgrp ^ (frow & 7)) * 16), g1 = g0 ^ 64u;
  const uint32_t ra = uint32_t(wm * kWM + frow) * 128u, rb = kStageA + uint32_t(wn * kWN + frow) * 128u;
  bf16x8_t fa0[kTM], fb0[kTN], fa1[kTM], fb1[kTN];
  auto read = [&](bf16x8_t (&fa)[kTM], bf16x8_t (&fb)[kTN], const uint8_t *stage, uint32_t g) {
#pragma unroll
    for (int i = 0; i < kTM; ++i)
      fa[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4 *>(stage + ra + i * 2048 + g));
#pragma unroll
    for (int j = 0; j < kTN; ++j)
      fb[j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4 *>(stage + rb + j * 2048 + g));
  };
  f32x4_t acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One 32-wide slice, its order pinned by scheduling barriers: the MFMAs of
  // (fa, fb); after every kPerRead of them one read of the next slice's
  // fragments (into na, nb, from stage `next`, granule offset g); and, with
  // kCopy, one of this wave's copies of step copy_kt into stage copy_stage
  // after every kCopyEvery MFMAs (spread over the slice; issuing them
  // together at its start measured the same).
  constexpr int kCopies = kDmaA + kDmaB;
  constexpr int kCopyEvery = kMfmas / kCopies > 0 ? kMfmas / kCopies : 1;
  // Decode positions (kWDec, first slice of a step): the lookups of chunk c
  // after MFMA c * kDecStep, its packing and store kDecGap MFMAs later; the
  // next codes' loads after the last store.
  constexpr int kDecStep = kDec > 0 ? (kMfmas * 3 / 4) / kDec : 1;
  constexpr int kDecGap = kDecStep / 2 > 0 ? kDecStep / 2 : 1;
  static_assert(!kWDec || (kDecGap <= kDecStep && (kDec - 1) * kDecStep + kDecGap + 1 < kMfmas),
                "each chunk packed before the next lookups; the next codes loaded within the slice");
  auto slice = [&](auto do_read, auto do_copy, auto do_decode, const bf16x8_t (&fa)[kTM],
                   const bf16x8_t (&fb)[kTN], bf16x8_t (&na)[kTM], bf16x8_t (&nb)[kTN], const uint8_t *next,
                   uint32_t g, int copy_kt, int copy_stage, uint8_t *dec_stage, int codes_kt) {
    constexpr bool kRead = decltype(do_read)::value, kCopy = decltype(do_copy)::value;
    constexpr bool kDecode = decltype(do_decode)::value;
    const uint32_t dst = __builtin_amdgcn_readfirstlane(lds0 + uint32_t(copy_stage) * kStage);
    const uint16_t *sa = a_split + size_t(copy_kt) * kBK, *sw = w_split + size_t(copy_kt) * kBK;
    if constexpr (kDecode) wait_vmcnt<kDmaA>();  // this step's codes (the A copy issued after them may fly on)
#pragma unroll
    for (int p = 0; p < kMfmas; ++p) {
      acc[p / kTN][p % kTN] =
          __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[p / kTN], fb[p % kTN], acc[p / kTN][p % kTN], 0, 0, 0);
      if constexpr (kRead) {
        if (p % kPerRead == kPerRead - 1 && p / kPerRead < kReads) {
          const int r = p / kPerRead;
          if (r < kTM)
            na[r] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4 *>(next + ra + r * 2048 + g));
          else
            nb[r - kTM] =
                __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4 *>(next + rb + (r - kTM) * 2048 + g));
        }
      }
      if constexpr (kCopy) {
        if (p % kCopyEvery == 0 && p / kCopyEvery < kCopies) {
          const int d = p / kCopyEvery;
          if (d < kDmaA)
            dma16_offset(sa, oa[d], dst + uint32_t(wave * kDmaA + d) * 1024u);
          else
            dma16_offset(sw, ob[d - kDmaA], dst + kStageA + uint32_t(wave * kDmaB + d - kDmaA) * 1024u);
        }
      }
      if constexpr (kDecode) {
        // A chunk's packing comes before the next chunk's lookups (one
        // register set holds the looked-up entries).
        if (p >= kDecGap && (p - kDecGap) % kDecStep == 0 && (p - kDecGap) / kDecStep < kDec)
          pack_store((p - kDecGap) / kDecStep, dec_stage);
        if (p % kDecStep == 0 && p / kDecStep < kDec) lookup(p / kDecStep);
        if (p == (kDec - 1) * kDecStep + kDecGap + 1) load_codes(codes_kt);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const std::true_type yes;
  const std::false_type no;

  // The loop body is free of branches (a branch there splits the
  // accumulators' live ranges into copies): the last step runs after it, and
  // the copy that the second-to-last step would issue for step KT repeats
  // step KT - 1 into the stage nobody reads any more.
  const int KT = ksteps;
  if constexpr (kWDec) {
    // Tile 0: codes and A copy; its codes decoded here (one code buffer, so
    // tile 1's codes are loaded after), then tile 1's codes and A copy.
    load_codes(0);
    copy(0, 0);
    wait_vmcnt<kDmaA>();
    lds_barrier();  // the table
#pragma unroll
    for (int c = 0; c < kDec; ++c) {
      lookup(c);
      pack_store(c, smem);
    }
    load_codes(min(1, KT - 1));
    copy(min(1, KT - 1), 1);
    wait_vmcnt<kDmaA + kDec>();  // tile 0's A copy
  } else {
    copy(0, 0);
    if (KT > 1) {
      copy(1, 1);
      wait_vmcnt<kDmaA + kDmaB>();
    } else {
      wait_vmcnt<0>();
    }
  }
  lds_barrier();
  read(fa0, fb0, smem, g0);
  for (int kt = 0; kt + 1 < KT; ++kt) {
    // Slice 0 of step kt (registers 0) while slice 1 is read (registers 1)
    // and (kWDec) the codes of tile kt + 1 are decoded into its stage.
    slice(yes, no, std::integral_constant<bool, kWDec>{}, fa0, fb0, fa1, fb1, smem + (kt & 1) * kStage, g1, 0, 0,
          smem + ((kt + 1) & 1) * kStage, min(kt + 2, KT - 1));
    // This wave's copy of step kt + 1 has landed (and its stores of the
    // decoded W) and its reads of stage kt & 1 are done; after the barrier
    // the same holds for every wave.  The codes of tile kt + 2 may fly on.
    wait_vmcnt<kDec>();
    lds_barrier();
    // Slice 1 of step kt while slice 0 of step kt + 1 is read and step
    // kt + 2 is copied into the stage step kt used.
    slice(yes, yes, no, fa1, fb1, fa0, fb0, smem + ((kt + 1) & 1) * kStage, g0, min(kt + 2, KT - 1), kt & 1, smem,
          0);
  }
  slice(yes, no, no, fa0, fb0, fa1, fb1, smem + ((KT - 1) & 1) * kStage, g1, 0, 0, smem, 0);
  slice(no, no, no, fa1, fb1, fa0, fb0, smem, g0, 0, 0, smem, 0);
  wait_vmcnt<0>();  // the repeated copy (and codes) of the last step

  if (partial) {
    store_tile<kTM, kTN>(acc, m0 + wm * kWM, n0 + wn * kWN, frow, fgrp, ts, cs, bias, bias_dtype, out, out_dtype,
                         M, N, partial, split);
    return;
  }
  lds_barrier();  // every wave is done reading the stages
  store_tile_lds<kTM, kTN>(acc, smem + wave * epilogue_region_bytes<kTM, kTN>(), m0 + wm * kWM, n0 + wn * kWN, lane,
                           ts, cs, bias, bias_dtype, out, out_dtype, M, N);
}

// Split-K epilogue: out = (sum over s of partial[s]) * ts[m] * cs[n] (+ b[n]),
// four consecutive columns per thread (N % 4 == 0), splits added in order.
// kS > 0: the split count is known, and all kS partial loads of a quad are
// issued before the first add (a loop over a run-time count waits for each
// load in turn: 4 splits of 512 x 4096 took 10.3 us); kS == 0 takes any count.
template <int kS>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(
    const float *__restrict__ partial, int splits, const float *__restrict__ ts,
    const float *__restrict__ cs, const void *__restrict__ bias, int bias_dtype,
    void *__restrict__ out, int out_dtype, int M, int N) {
  const uint32_t quads = uint32_t(M) * uint32_t(N / 4);  // plan_gemm splits only when this fits 32 bits
  const size_t plane = size_t(M) * N;
  for (uint32_t q = blockIdx.x * 256u + threadIdx.x; q < quads; q += gridDim.x * 256u) {
    const uint32_t row = q / uint32_t(N / 4), col = (q - row * uint32_t(N / 4)) * 4u;
    const size_t e0 = size_t(q) * 4;
    f32x4_t sum;
    if constexpr (kS > 0) {
      f32x4_t v[kS];
#pragma unroll
      for (int s = 0; s < kS; ++s) v[s] = *reinterpret_cast<const f32x4_t *>(partial + s * plane + e0);
      sum = v[0];
#pragma unroll
      for (int s = 1; s < kS; ++s) sum += v[s];
    } else {
      sum = *reinterpret_cast<const f32x4_t *>(partial + e0);
      for (int s = 1; s < splits; ++s) sum += *reinterpret_cast<const f32x4_t *>(partial + s * plane + e0);
    }
    const float t = ts[row];
    uint16_t h[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float b = 0.f;
      if (bias) {
        const uint16_t hb = static_cast<const uint16_t *>(bias)[col + c];
        b = bias_dtype == HIF8_DTYPE_BF16 ? half_bits_to_float<true>(hb) : half_bits_to_float<false>(hb);
      }
      const float y = sum[c] * t * cs[col + c] + b;
      h[c] = out_dtype == HIF8_DTYPE_BF16 ? float_to_bf16_bits(y) : float_to_f16_bits(y);
    }
    uint16_t *o = static_cast<uint16_t *>(out) + e0;
    *reinterpret_cast<uint2 *>(o) = make_uint2(uint32_t(h[0]) | (uint32_t(h[1]) << 16),
                                               uint32_t(h[2]) | (uint32_t(h[3]) << 16));
  }
}

// The split-K reduce of a launch with `splits` partial planes.
void launch_splitk_reduce(const LinearArgs &a, const float *partial, int splits) {
  const size_t quads = size_t(a.m) * size_t(a.n / 4);
  const unsigned blocks = unsigned(std::min<size_t>((quads + 255) / 256, 4096));
  auto go = [&](auto kern) {
    kern<<<blocks, 256, 0, a.stream>>>(partial, splits, a.act_scale, a.channel_scale, a.bias, a.bias_dtype, a.out,
                                       a.out_dtype, int(a.m), int(a.n));
  };
  switch (splits) {
    case 2: go(splitk_reduce_kernel<2>); break;
    case 4: go(splitk_reduce_kernel<4>); break;
    case 8: go(splitk_reduce_kernel<8>); break;
    default: go(splitk_reduce_kernel<0>); break;
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

// Block shape, K split and workspace layout of a tiled launch.  256 x 256
// blocks of 8 waves run at the highest rate per CU but need >= 128 tiles;
// smaller grids use 128 x 128 blocks of 4 waves (two per CU).  When the tiles
// still leave CUs idle, K is split in powers of two while every split keeps
// >= 16 K steps, up to about one block per CU slot.  The workspace holds the
// bf16 copy of A (M x K x 2 bytes, 256-byte aligned) and then the split
// partials (splits x M x N x 4 bytes).
struct GemmPlan {
  int tile;          // 256 (8 waves) or 128 (4 waves)
  int bn;            // block columns: tile, or 192 for 256-row tiles (decoded weights only)
  int splits;        // K splits
  bool w_pre;        // W decoded once per call too (large M)
  size_t a_bytes;    // bf16 copy of A
  size_t w_bytes;    // bf16 copy of W (0 unless w_pre)
  size_t part_bytes; // FP32 partials (0 when unsplit)
};

int env_int(const char *name, int fallback) {
  const char *v = getenv(name);
  return v && *v ? atoi(v) : fallback;
}

// decoded_weight: the plan of soft_hif8_gemm_decoded_weight, whose kernel
// reads W by DMA at every M.  There, from M = 2048 on, a grid of at most 128
// 256-tiles (half the CUs) runs faster as unsplit 128-tiles than as 256-tiles
// split in two (4096 x 2048 x 4096: 88 vs 99.5 us on MI355X); with 192 tiles
// (M = 512 gate_up) 256-tiles win.
GemmPlan plan_gemm(int64_t m, int64_t n, int64_t k, bool decoded_weight = false) {
  static const int tile_env = env_int("HIF8_GEMM_TILE", 0);
  static const int split_env = env_int("HIF8_GEMM_SPLIT", 0);
  static const int wpre_env = env_int("HIF8_GEMM_WPRE", -1);
  // Decoding W once costs ~3 bytes of HBM traffic per weight; the in-kernel
  // decode repeats it once per 256-row tile of M, so from M = 2048 on the
  // codes path decodes W once per call into the workspace and runs the plan
  // of the decoded-weight path (both operands by DMA).
  if (!decoded_weight && (wpre_env >= 0 ? wpre_env > 0 : m >= 2048) && k < kMaxDmaK && k % kBK == 0) {
    GemmPlan p = plan_gemm(m, n, k, true);
    p.w_pre = true;
    p.w_bytes = (size_t(n) * size_t(k) * 2 + 255) / 256 * 256;
    return p;
  }
  GemmPlan p;
  const int64_t tiles256 = ((m + 255) / 256) * ((n + 255) / 256);
  const int64_t ksteps = k / kBK;
  const bool splittable = n % 4 == 0 && k % kBK == 0 && m * (n / 4) <= int64_t(0xFFFFFFFFll);
  // 256-tiles also when a K split of >= 24 steps each fills all 256 CUs
  // exactly (long K, e.g. the down projection at M = 512): their 8-wave
  // blocks run faster per step than two 4-wave 128-tile blocks.
  int64_t s256 = 1;
  while (splittable && tiles256 * s256 * 2 <= 256 && ksteps % (s256 * 2) == 0 && ksteps / (s256 * 2) >= 24)
    s256 *= 2;
  const bool long_k_fill = m >= 256 && tiles256 * s256 == 256;
  p.tile = tile_env == 128 || tile_env == 256 ? tile_env
                                              : (m >= 256 && (tiles256 >= 128 || long_k_fill) ? 256 : 128);
  // ... unless 256 x 128 blocks fill the CUs in one wave without a split:
  // 8 waves per CU either way, but one block shares its A panel over 128
  // columns instead of two 128 x 128 blocks each copying their own.
  static const int bn128_env = env_int("HIF8_GEMM_BN128", 1);
  const int64_t tiles256x128 = ((m + 255) / 256) * ((n + 127) / 128);
  const bool bn128 = decoded_weight && tile_env == 0 && m >= 2048 && tiles256 <= 128 && bn128_env &&
                     tiles256x128 > 128 && tiles256x128 <= 256;
  if (decoded_weight && tile_env == 0 && m >= 2048 && tiles256 <= 128 && !bn128) p.tile = 128;
  const int64_t tiles = ((m + p.tile - 1) / p.tile) * ((n + p.tile - 1) / p.tile);
  const int64_t slots = p.tile == 256 ? 256 : 512;  // resident blocks on 256 CUs
  p.splits = 1;
  if (splittable) {
    if (split_env > 0) {
      while (p.splits * 2 <= split_env && ksteps % (p.splits * 2) == 0) p.splits *= 2;
    } else if (p.tile == 256 && tiles256 < 128) {
      p.splits = int(s256);
    } else {
      while (tiles * p.splits * 2 <= slots && ksteps % (p.splits * 2) == 0 && ksteps / (p.splits * 2) >= 16)
        p.splits *= 2;
    }
  }
  // Decoded weights: an unsplit 256-tile grid short of one block per CU
  // takes 256 x 192 blocks when those still fit one wave of blocks (gate_up
  // at M = 512: 192 -> 256 blocks).  The in-kernel weight decode does not
  // divide over 192 rows, so the code path keeps 256 x 256.
  p.bn = p.tile;
  if (bn128) {
    p.splits = 1;
    p.bn = 128;
  }
  if (decoded_weight && p.tile == 256 && p.splits == 1 && tile_env == 0 && !bn128) {
    const int64_t tiles192 = ((m + 255) / 256) * ((n + 191) / 192);
    if (tiles256 < 256 && tiles192 > tiles256 && tiles192 <= 256) p.bn = 192;
  }
  // Codes path below M = 2048: 256 x 128 blocks of the DMA kernel with the
  // weight decoded in it, K split in powers of two (>= 16 steps each) until
  // the grid is one block per CU, where that fills all 256 CUs (knob
  // HIF8_GEMM_WDEC128=0 turns it off).  Measured on MI355X at M = 512
  // against the 128 x 128 / 256 x 256 plans above: q and o 4096 x 4096 41
  // vs 43-44 us, down 4096 x 12288 78.7 vs 80.4-81.5; k/v (128 blocks)
  // 35.2 vs 31.6, so it keeps the plan above.
  static const int wdec128_env = env_int("HIF8_GEMM_WDEC128", 1);
  if (!decoded_weight && wdec128_env && tile_env == 0 && split_env == 0 && splittable && m >= 256 &&
      k < kMaxDmaK && (tiles256 < 128 || long_k_fill)) {
    const int64_t t128 = ((m + 255) / 256) * ((n + 127) / 128);
    int s128 = 1;
    while (t128 * s128 * 2 <= 256 && ksteps % (s128 * 2) == 0 && ksteps / (s128 * 2) >= 16) s128 *= 2;
    if (t128 * s128 == 256) {
      p.tile = 256;
      p.bn = 128;
      p.splits = s128;
    }
  }
  p.w_pre = false;
  p.a_bytes = (size_t(m) * size_t(k) * 2 + 255) / 256 * 256;
  p.w_bytes = p.w_pre ? (size_t(n) * size_t(k) * 2 + 255) / 256 * 256 : 0;
  p.part_bytes = p.splits > 1 ? size_t(p.splits) * size_t(m) * size_t(n) * sizeof(float) : 0;
  return p;
}

template <int kBM, int kBN, int kWavesM, int kWavesN, bool kAPre, bool kPingPong>
int launch_tiled(const LinearArgs &a, const void *act, const void *wt, int splits, float *partial) {
  // K-step stages, or the epilogue regions if larger; + 512 B of static LDS (the table).
  constexpr size_t kSmem = std::max<size_t>(2 * size_t(kBM + kBN) * kBK * 2,
                                            size_t(kWavesM * kWavesN) *
                                                epilogue_region_bytes<kBM / kWavesM / 16, kBN / kWavesN / 16>());
  constexpr int kT = kWave * kWavesM * kWavesN;
  if (const int st = reserve_dynamic_lds(
          reinterpret_cast<const void *>(&gemm_kernel<kBM, kBN, kWavesM, kWavesN, kAPre, kPingPong>), kSmem,
          "soft_hif8 GEMM"))
    return st;
  const int64_t tiles = ((a.n + kBN - 1) / kBN) * ((a.m + kBM - 1) / kBM);
  const dim3 grid(unsigned((tiles * splits + 7) / 8 * 8));
  gemm_kernel<kBM, kBN, kWavesM, kWavesN, kAPre, kPingPong><<<grid, kT, kSmem, a.stream>>>(
      act, a.act_scale, wt, a.channel_scale, a.bias, a.bias_dtype, a.out, a.out_dtype, int(a.m),
      int(a.n), int(a.k), partial, splits, int(a.k / kBK / splits));
  int st = check_launch("soft_hif8 GEMM");
  if (st || !partial) return st;
  launch_splitk_reduce(a, partial, splits);
  return check_launch("soft_hif8 GEMM (split-K reduce)");
}

// Launch of gemm_dma_kernel (+ the split-K reduce when partial is set); wt
// is the bf16 weight, or (kWDec) the codes.
template <int kBM, int kBN, int kWavesM, int kWavesN, bool kWDec = false>
int launch_dma(const LinearArgs &a, const uint16_t *act, const void *wt, int splits, float *partial) {
  constexpr size_t kSmem = std::max<size_t>(2 * size_t(kBM + kBN) * kBK * 2,
                                            size_t(kWavesM * kWavesN) *
                                                epilogue_region_bytes<kBM / kWavesM / 16, kBN / kWavesN / 16>());
  constexpr int kT = kWave * kWavesM * kWavesN;
  if (const int st = reserve_dynamic_lds(
          reinterpret_cast<const void *>(&gemm_dma_kernel<kBM, kBN, kWavesM, kWavesN, kWDec>), kSmem,
          "soft_hif8 GEMM"))
    return st;
  const int64_t tiles = ((a.n + kBN - 1) / kBN) * ((a.m + kBM - 1) / kBM);
  const dim3 grid(unsigned((tiles * splits + 7) / 8 * 8));
  gemm_dma_kernel<kBM, kBN, kWavesM, kWavesN, kWDec><<<grid, kT, kSmem, a.stream>>>(
      act, a.act_scale, wt, a.channel_scale, a.bias, a.bias_dtype, a.out, a.out_dtype, int(a.m), int(a.n),
      int(a.k), partial, splits, int(a.k / kBK / splits));
  int st = check_launch("soft_hif8 GEMM");
  if (st || !partial) return st;
  launch_splitk_reduce(a, partial, splits);
  return check_launch("soft_hif8 GEMM (split-K reduce)");
}

// Both operands bf16 in HBM: the DMA-fed kernel with the plan's block shape.
int launch_bf16_operands(const LinearArgs &a, const GemmPlan &p, const uint16_t *act, const uint16_t *wt, int splits,
                         float *partial) {
  if (a.k >= kMaxDmaK) return fail(HIF8_ERR_UNSUPPORTED, "soft_hif8 GEMM: K >= %d", kMaxDmaK);
  if (p.tile == 256 && p.bn == 192) return launch_dma<256, 192, 4, 2>(a, act, wt, splits, partial);
  if (p.tile == 256 && p.bn == 128) return launch_dma<256, 128, 4, 2>(a, act, wt, splits, partial);
  if (p.tile == 256) return launch_dma<256, 256, 4, 2>(a, act, wt, splits, partial);
  return launch_dma<128, 128, 2, 2>(a, act, wt, splits, partial);
}

template <bool kAPre>
int launch_plan(const LinearArgs &a, const GemmPlan &p, const void *act, int splits, float *partial) {
  static const int pingpong = env_int("HIF8_GEMM_PINGPONG", 1);
  // An unsplit 256-tile grid short of one block per CU that 256 x 192 blocks
  // fill in one wave (gate_up at M = 512: 192 -> 256 blocks) runs the DMA
  // kernel with the weight decoded in it (142 -> 111 us there; at 256 x 256
  // it measured no faster than the ping-pong kernel).
  if (kAPre && p.tile == 256 && p.bn == 128)
    return launch_dma<256, 128, 4, 2, true>(a, static_cast<const uint16_t *>(act), a.weight, splits, partial);
  const int64_t tiles_m = (a.m + 255) / 256, t256 = tiles_m * ((a.n + 255) / 256), t192 = tiles_m * ((a.n + 191) / 192);
  if (kAPre && p.tile == 256 && splits == 1 && a.k < kMaxDmaK && t256 < 256 && t192 > t256 && t192 <= 256)
    return launch_dma<256, 192, 4, 2, true>(a, static_cast<const uint16_t *>(act), a.weight, splits, partial);
  if (p.tile == 256)
    return pingpong ? launch_tiled<256, 256, 2, 4, kAPre, true>(a, act, a.weight, splits, partial)
                    : launch_tiled<256, 256, 2, 4, kAPre, false>(a, act, a.weight, splits, partial);
  return launch_tiled<128, 128, 2, 2, kAPre, false>(a, act, a.weight, splits, partial);
}

}  // namespace

size_t gemm_workspace_size(int64_t m, int64_t n, int64_t k) {
  if (m <= 4 || m > 0x7FFFFFFFll || n > 0x7FFFFFFFll || k > 0x7FFFFFFFll || n <= 0 || k <= 0 || k % kBK)
    return 0;
  const GemmPlan p = plan_gemm(m, n, k);
  return p.a_bytes + p.w_bytes + p.part_bytes;
}

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
  const GemmPlan p = plan_gemm(a.m, a.n, a.k);
  const bool use_ws = a.workspace && a.workspace_bytes >= p.a_bytes + p.w_bytes + p.part_bytes &&
                      aligned(a.workspace, 256);
  if (!use_ws) return launch_plan<false>(a, p, a.act, 1, nullptr);
  uint8_t *ws = static_cast<uint8_t *>(a.workspace);
  uint16_t *abf = reinterpret_cast<uint16_t *>(ws);
  const size_t chunks = size_t(a.m) * size_t(a.k) / 16;
  // The activation, and with w_pre the weight too, in one launch.
  uint16_t *wbf = p.w_pre ? reinterpret_cast<uint16_t *>(ws + p.a_bytes) : nullptr;
  const size_t wchunks = p.w_pre ? size_t(a.n) * size_t(a.k) / 16 : 0;
  const unsigned blocks = unsigned(std::min<size_t>((chunks + wchunks + 255) / 256, p.w_pre ? 4096 : 2048));
  decode_rows_kernel<<<blocks, 256, 0, a.stream>>>(static_cast<const uint8_t *>(a.act), abf, chunks, a.weight, wbf,
                                                   wchunks);
  const int st = check_launch(p.w_pre ? "soft_hif8 GEMM (activation and weight decode)"
                                      : "soft_hif8 GEMM (activation decode)");
  if (st) return st;
  float *partial = p.part_bytes ? reinterpret_cast<float *>(ws + p.a_bytes + p.w_bytes) : nullptr;
  if (p.w_pre) {
    const uint16_t *wbf = reinterpret_cast<const uint16_t *>(ws + p.a_bytes);
    return launch_bf16_operands(a, p, abf, wbf, p.part_bytes ? p.splits : 1, partial);
  }
  return launch_plan<true>(a, p, abf, p.part_bytes ? p.splits : 1, partial);
}

size_t gemm_decoded_weight_workspace_size(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || m > 0x7FFFFFFFll || n > 0x7FFFFFFFll || k > 0x7FFFFFFFll || k % kBK)
    return 0;
  const GemmPlan p = plan_gemm(m, n, k, true);
  return p.a_bytes + p.part_bytes;
}

int launch_gemm_decoded_weight(const LinearArgs &a) {
  const GemmPlan p = plan_gemm(a.m, a.n, a.k, true);
  uint8_t *ws = static_cast<uint8_t *>(a.workspace);
  uint16_t *abf = reinterpret_cast<uint16_t *>(ws);
  const size_t chunks = size_t(a.m) * size_t(a.k) / 16;
  decode_rows_kernel<<<unsigned(std::min<size_t>((chunks + 255) / 256, 2048)), 256, 0, a.stream>>>(
      static_cast<const uint8_t *>(a.act), abf, chunks, nullptr, nullptr, 0);
  const int st = check_launch("soft_hif8 GEMM (activation decode)");
  if (st) return st;
  float *partial = p.part_bytes ? reinterpret_cast<float *>(ws + p.a_bytes) : nullptr;
  return launch_bf16_operands(a, p, abf, a.weight_bf16, p.part_bytes ? p.splits : 1, partial);
}

int launch_decode_bf16(const uint8_t *codes, uint16_t *out, size_t elements, hipStream_t stream) {
  const size_t chunks = elements / 16;
  decode_rows_kernel<<<unsigned(std::min<size_t>((chunks + 255) / 256, 4096)), 256, 0, stream>>>(
      codes, out, chunks, nullptr, nullptr, 0);
  return check_launch("hif8_decode_bf16");
}

}  // namespace hif8
