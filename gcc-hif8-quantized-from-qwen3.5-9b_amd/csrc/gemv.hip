// Decode GEMV (m <= 4) for gfx950: y[m, n] = sum_k dec(a[m,k]) dec(w[n,k]) * ts[m] * cs[n] (+ b[n]).
//
// The weight stream (n*k bytes) dominates and is read exactly once, so the
// kernel is built to keep HBM busy with little VALU work per byte:
//   * a block of 256 threads owns kR consecutive weight rows; thread t owns the
//     16-byte column chunk t (+256 per segment), so each wavefront load covers
//     1 KiB of contiguous row bytes and a thread has kR 16-byte loads in flight;
//   * the activation chunk (m <= 4 rows) is decoded once per chunk into packed
//     bf16 pairs and stays in VGPRs for all kR weight rows;
//   * weight bytes are decoded with a bf16 table in LDS (HiF8 is a subset of
//     bf16, so decode is exact; replicated per lane for small grids, see
//     RepLut) and multiplied with v_dot2_f32_bf16, FP32 accumulation;
//   * each wavefront sums its kR*kM partials over its 64 lanes in registers
//     (permlane swaps and DPP, halving the values per lane at each level),
//     the four wavefront totals meet in LDS, and the epilogue applies token
//     scale, channel scale and bias, rounding once.
// The fused variants take fp16/bf16 x and encode it on the fly: with the
// fixed scale (soft_hif8_fused_gemm.cpp:449-534 with HIF8_FUSED_STATIC_SCALE)
// or with each row's dynamic scale max(finite amax, 1e-12), which every block
// reduces from the whole row first (soft_hif8_fused_gemm.cpp:536-571).
#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

#include "linear.h"

namespace hif8 {
namespace {

constexpr int kThreads = 256;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Decode-table lookups.  LDS serves a DS instruction 32 lanes at a time from
// 32 four-byte banks.  The plain 256-entry bf16 table (CompactLut) spans 128
// dwords, four per bank, and lanes holding codes in different dwords of one
// bank are served one after another: measured on MI355X, a wavefront of
// lookups takes 2.3x the conflict-free time for codes quantised from Gaussian
// weights (1.7x for codes uniform in 0..110).
//
// RepLut is the conflict-free form: code c owns the 128-byte row at byte
// 256 c, 32 dwords each holding bf16(dec(c)) in both halves, and lane l reads
// dword l % 32 of the row, so the 32 lanes served together always hit 32
// distinct banks.  The address is one v_perm_b32 of the code byte and the
// lane's column, as the plain table's is one shift; but the table takes 64 KiB
// of LDS (half of it unused), which leaves room for two blocks per CU.  The
// GEMV therefore uses it only when its grid fits the chip in one round of two
// blocks per CU (kRepMaxBlocks): there the blocks' latency sets the time and
// the faster lookups shorten it (MI355X, graphs of 20 launches over >= 768 MB
// of weights quantised from Gaussian rows, M = 1: q 4096 x 4096 5.27 vs 5.50
// us, k+v 3.98 vs 4.18, o 5.36 vs 5.59; M = 4: down 4096 x 12288 13.6 vs
// 14.4).  Larger grids
// stream as fast as the memory pipeline allows with four blocks per CU and
// the plain table, and lose 5-10 % with the big one (gate_up 24576 x 4096, M
// = 4: 22.0-22.9 vs 20.6-21.0 us, also as 512-thread blocks of two 4-wave
// teams sharing one table), though their lookups wait far less (rocprofv3
// SQ_WAIT_INST_LDS down 3x, SQ_LDS_BANK_CONFLICT 0).
constexpr uint32_t kRepLutBytes = 256 * 256;
constexpr int64_t kRepMaxBlocks = 2 * 256;

struct RepLut {
  const uint8_t *t;  // LDS, kRepLutBytes
  uint32_t col;      // 4 * (lane % 32)
  // Entry of byte kByte of the word w.
  template <int kByte>
  __device__ __forceinline__ uint16_t byte(uint32_t w) const {
    const uint32_t off = __builtin_amdgcn_perm(col, w, 0x0C0C0004u | (uint32_t(kByte) << 8));
    return *reinterpret_cast<const uint16_t *>(t + off);
  }
  __device__ __forceinline__ uint16_t code(uint32_t c) const { return byte<0>(c); }
};

struct CompactLut {
  const uint16_t *t;  // LDS, 256 entries, at LDS address 0 (a lookup address is one shift of the byte)
  template <int kByte>
  __device__ __forceinline__ uint16_t byte(uint32_t w) const { return t[(w >> (8 * kByte)) & 0xFFu]; }
  __device__ __forceinline__ uint16_t code(uint32_t c) const { return t[c]; }
};

// Entry `tid` of the decode table: bf16 bits of dec(tid).
__device__ __forceinline__ uint32_t decode_entry(int tid) { return decode_bits(uint32_t(tid)) >> 16; }

// The decode table of a block of 256 threads, in LDS at `tab` (kRep: RepLut,
// else CompactLut); thread t passes e = decode_entry(t).  Replicated, thread t
// writes row t as eight 16-byte stores at column quads rotated by t, so the
// lanes of one store instruction cover distinct banks.
template <bool kRep>
__device__ __forceinline__ void fill_decode_table(uint8_t *tab, int tid, uint32_t e) {
  if constexpr (kRep) {
    const uint32_t v = e | (e << 16);
    u32x4 *row = reinterpret_cast<u32x4 *>(tab + 256u * uint32_t(tid));
#pragma unroll
    for (int j = 0; j < 8; ++j) row[(j + tid) & 7] = u32x4{v, v, v, v};
  } else {
    reinterpret_cast<uint16_t *>(tab)[tid] = uint16_t(e);
  }
}

template <bool kRep>
using DecodeLut = std::conditional_t<kRep, RepLut, CompactLut>;

template <bool kRep>
__device__ __forceinline__ DecodeLut<kRep> decode_lut(const uint8_t *tab, int lane) {
  if constexpr (kRep) return RepLut{tab, 4u * uint32_t(lane & 31)};
  else return CompactLut{reinterpret_cast<const uint16_t *>(tab)};
}

// 16 HiF8 bytes -> 8 packed bf16 pairs (each pair packs with one v_perm_b32).
template <class Lut>
__device__ __forceinline__ void decode16(const Lut &lut, const u32x4 q, uint32_t (&p)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = q[i];
    u16x2 lo, hi;
    lo.x = lut.template byte<0>(w);
    lo.y = lut.template byte<1>(w);
    hi.x = lut.template byte<2>(w);
    hi.y = lut.template byte<3>(w);
    p[2 * i] = __builtin_bit_cast(uint32_t, lo);
    p[2 * i + 1] = __builtin_bit_cast(uint32_t, hi);
  }
}

__device__ __forceinline__ bool near_index_boundary(float q) {
  const uint32_t u = __float_as_uint(q);
  return (((u + 8u) & 0x7FFFFu) <= 16u) || __builtin_isnan(q);
}

// Static encode (fixed scale) + decode of 16 fp16/bf16 values into bf16 pairs.
// Multiplies by the reciprocal and redoes the element with an IEEE division
// when the product is within 8 ulps of an encode-index boundary or NaN (the
// same rule as hif8_static_quant), so the codes equal the standalone quant's.
// Two LDS lookups per element (encode table, decode table): measured on
// MI355X, rounding the quotient's bits arithmetically instead (about 20 VALU
// operations per element) made the fused GEMV 20-30 % slower, since every
// block re-encodes its activation chunk.
// All 16 take the multiply first; one branch (rarely taken) redoes the 16
// with the division, so the kernel holds one copy of the division code per
// 16 values instead of one per pair.
template <bool kBf16, class Lut>
__device__ __forceinline__ void fast_encode_decode16(const u32x4 a, const u32x4 b, float s, float r,
                                                     const uint8_t *enc, const Lut &dec, u32x4 &lo,
                                                     u32x4 &hi) {
  uint32_t u[16];
  bool redo = false;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = i < 4 ? a[i] : b[i - 4];
    const float q0 = lo_to_float<kBf16>(w) * r, q1 = hi_to_float<kBf16>(w) * r;
    redo |= near_index_boundary(q0) | near_index_boundary(q1);
    u[2 * i] = __float_as_uint(q0);
    u[2 * i + 1] = __float_as_uint(q1);
  }
  if (__builtin_expect(redo, 0)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = i < 4 ? a[i] : b[i - 4];
      const float q0 = lo_to_float<kBf16>(w) / s, q1 = hi_to_float<kBf16>(w) / s;
      // NaN quotients index an entry of exponent 0xFF whose top mantissa bit
      // is set, which encodes to the NaN code.
      u[2 * i] = __builtin_isnan(q0) ? 0x7FC00000u : __float_as_uint(q0);
      u[2 * i + 1] = __builtin_isnan(q1) ? 0x7FC00000u : __float_as_uint(q1);
    }
  }
  uint32_t p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    p[i] = uint32_t(dec.code(enc[u[2 * i] >> 19])) | (uint32_t(dec.code(enc[u[2 * i + 1] >> 19])) << 16);
  lo = u32x4{p[0], p[1], p[2], p[3]};
  hi = u32x4{p[4], p[5], p[6], p[7]};
}

// Quantise-dequantise table of the fused static kinds in the MFMA-4 GEMV:
// entry i (the 13-bit sign / exponent / top-four-mantissa index of an FP32
// quotient x / s, the index of Tables::static_encode) holds the bf16 bits of
// dec(static_encode[i]).  One lookup instead of the encode and decode lookups;
// 16 KiB, copied into LDS by each block.
struct QdqTable {
  uint16_t v[8192];
};

constexpr QdqTable make_qdq_table() {
  QdqTable t{};
  for (uint32_t i = 0; i < 8192; ++i) t.v[i] = uint16_t(decode_bits(static_encode_bits(i << 19)) >> 16);
  return t;
}

static __device__ const QdqTable kQdqTable = make_qdq_table();

// Static encode + decode of 16 fp16/bf16 values into bf16 pairs through the
// quantise-dequantise table: the same reciprocal multiply, boundary test and
// IEEE-division redo as fast_encode_decode16, so each value equals
// dec(the standalone quant's code).  All 16 take the multiply first; one
// branch (rarely taken: a quotient within 8 ulps of an index boundary, or
// NaN) redoes the 16 with the division, so the kernel holds one copy of the
// division code per 16 values instead of one per pair.
template <bool kBf16>
__device__ __forceinline__ void fast_qdq16(const u32x4 a, const u32x4 b, float s, float r, const uint16_t *qdq,
                                           uint32_t (&p)[8]) {
  uint32_t u[16];
  bool redo = false;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t w = i < 4 ? a[i] : b[i - 4];
    const float q0 = lo_to_float<kBf16>(w) * r, q1 = hi_to_float<kBf16>(w) * r;
    redo |= near_index_boundary(q0) | near_index_boundary(q1);
    u[2 * i] = __float_as_uint(q0);
    u[2 * i + 1] = __float_as_uint(q1);
  }
  if (__builtin_expect(redo, 0)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = i < 4 ? a[i] : b[i - 4];
      const float q0 = lo_to_float<kBf16>(w) / s, q1 = hi_to_float<kBf16>(w) / s;
      // NaN quotients index the NaN entries of exponent 0xFF.
      u[2 * i] = __builtin_isnan(q0) ? 0x7FC00000u : __float_as_uint(q0);
      u[2 * i + 1] = __builtin_isnan(q1) ? 0x7FC00000u : __float_as_uint(q1);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = uint32_t(qdq[u[2 * i] >> 19]) | (uint32_t(qdq[u[2 * i + 1] >> 19]) << 16);
}

constexpr int pow2_floor(int v) {
  int p = 1;
  while (p * 2 <= v) p *= 2;
  return p;
}

constexpr int pow2_ceil(int v) {
  int p = 1;
  while (p < v) p *= 2;
  return p;
}

constexpr int log2_exact(int v) { return v <= 1 ? 0 : 1 + log2_exact(v / 2); }

// One exchange level of the in-register transpose-reduce, on lane bit kBit
// (5 = lanes l and l^32, 4 = 16-lane rows, 3..0 = DPP partners inside a row:
// mirror, half mirror, quad reverse, quad swap).  Every partner differs from
// its lane in bit kBit, so lanes whose bit is 0 end with lo + the partner's lo
// and lanes whose bit is 1 with hi + the partner's hi; called with lo == hi,
// every lane ends with the sum over the pair.
template <int kBit>
__device__ __forceinline__ float exchange_add(float lo, float hi, int lane) {
  if constexpr (kBit >= 4) {
    const auto s = kBit == 5 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false)
                             : __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
  } else {
    constexpr int kCtrl = kBit == 3 ? 0x140 : kBit == 2 ? 0x141 : kBit == 1 ? 0x1B : 0xB1;
    const bool up = (lane >> kBit) & 1;
    const float keep = up ? hi : lo, send = up ? lo : hi;
    return keep + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(send), kCtrl, 0xF, 0xF, false));
  }
}

// Sums v[0..kV) (kV a power of two <= 64) over the 64 lanes of a wavefront
// in log2(kV) halving levels plus 6 - log2(kV) full levels: 2 kV - 2 + 6 -
// log2(kV) lane exchanges instead of a round trip through LDS.  Afterwards
// lane l holds the total of index l >> (6 - log2(kV)).
template <int kV>
__device__ __forceinline__ float wave_transpose_sum(float (&v)[kV], int lane) {
  constexpr int kLevels = log2_exact(kV);
  static_assert((1 << kLevels) == kV && kV <= 64, "value count must be a power of two <= 64");
#pragma unroll
  for (int level = 0; level < kLevels; ++level) {
    const int half = kV >> (level + 1);
#pragma unroll
    for (int i = 0; i < half; ++i) {
      switch (5 - level) {
        case 5: v[i] = exchange_add<5>(v[i], v[i + half], lane); break;
        case 4: v[i] = exchange_add<4>(v[i], v[i + half], lane); break;
        case 3: v[i] = exchange_add<3>(v[i], v[i + half], lane); break;
        case 2: v[i] = exchange_add<2>(v[i], v[i + half], lane); break;
        case 1: v[i] = exchange_add<1>(v[i], v[i + half], lane); break;
        default: v[i] = exchange_add<0>(v[i], v[i + half], lane); break;
      }
    }
  }
  float s = v[0];
#pragma unroll
  for (int bit = 5 - kLevels; bit >= 0; --bit) {
    switch (bit) {
      case 5: s = exchange_add<5>(s, s, lane); break;
      case 4: s = exchange_add<4>(s, s, lane); break;
      case 3: s = exchange_add<3>(s, s, lane); break;
      case 2: s = exchange_add<2>(s, s, lane); break;
      case 1: s = exchange_add<1>(s, s, lane); break;
      default: s = exchange_add<0>(s, s, lane); break;
    }
  }
  return s;
}

__device__ __forceinline__ float load_bias(const void *bias, int dtype, int i) {
  const uint16_t h = static_cast<const uint16_t *>(bias)[i];
  return dtype == HIF8_DTYPE_BF16 ? half_bits_to_float<true>(h) : half_bits_to_float<false>(h);
}

__device__ __forceinline__ void store_out(void *out, int dtype, size_t i, float y) {
  static_cast<uint16_t *>(out)[i] =
      dtype == HIF8_DTYPE_BF16 ? float_to_bf16_bits(y) : float_to_f16_bits(y);
}

// The causal-conv epilogue (GemvConv) of output (m, c), y its fp32 value
// before the bf16 store.  Loads take clamped tap indices so they issue
// together; the taps past kw are read and ignored.
__device__ __forceinline__ void conv_epilogue(const GemvConv &cv, int m, int c, float y) {
  const uint32_t xb = float_to_bf16_bits(y);
  uint16_t *st = cv.state + (size_t(m) * cv.channels + c) * (cv.kw - 1);
  const uint16_t *w = cv.weight + size_t(c) * cv.kw;
  uint32_t sv[3], wv[4];
#pragma unroll
  for (int t = 0; t < 3; ++t) sv[t] = st[min(t, cv.kw - 2)];
#pragma unroll
  for (int t = 0; t < 4; ++t) wv[t] = w[min(t, cv.kw - 1)];
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < 3; ++t)
    if (t < cv.kw - 1) acc += half_bits_to_float<true>(sv[t]) * half_bits_to_float<true>(wv[t]);
  const uint32_t wl = cv.kw == 2 ? wv[1] : cv.kw == 3 ? wv[2] : wv[3];
  acc += half_bits_to_float<true>(xb) * half_bits_to_float<true>(wl);
#pragma unroll
  for (int t = 0; t < 2; ++t)
    if (t + 1 < cv.kw - 1) st[t] = uint16_t(sv[t + 1]);
  st[cv.kw - 2] = uint16_t(xb);
  cv.out[size_t(m) * cv.channels + c] = acc / (1.f + expf(-acc));
}

// Waves per SIMD the register allocation must allow.  Tighter bounds than
// these make the compiler spill (M = 2 at 5 waves, M = 4 at 4 waves).
constexpr int gemv_min_waves(int m, int rows) { return rows > 8 ? 2 : m == 1 ? 6 : m == 2 ? 4 : 2; }

// kOneChunk: k <= 16 * kThreads, so each thread owns at most one 16-byte
// column chunk per row (code activations or a fixed activation scale).
//
// act and weight carry no __restrict__: as restrict read-only operands their
// loads count as invariant, and the compiler sinks the one-chunk preload below
// the LDS barrier to its first use, serialising the set-up and the weight
// fetch that the preload exists to overlap.
template <int kM, int kR, int kSrc, bool kOneChunk, bool kRep>
__global__ __launch_bounds__(kThreads, gemv_min_waves(kM, kR)) void gemv_kernel(
    const void *act, const float *__restrict__ act_scale,
    const uint8_t *weight, const float *__restrict__ cs,
    const void *__restrict__ bias, int bias_dtype, void *__restrict__ out, int out_dtype,
    int n, int k, const GemvPair pair, const GemvConv conv) {
  constexpr int kV = kR * kM;
  constexpr int kVp = pow2_ceil(kV);  // partial sums per lane, zero-padded
  constexpr int kWaves = kThreads / kWave;
  constexpr bool kFused = kSrc != kActCodes;
  constexpr bool kDynamic = kSrc == kActF16Dyn || kSrc == kActBf16Dyn;
  constexpr bool kInBf16 = kSrc == kActBf16 || kSrc == kActBf16Dyn;
  constexpr int kActWords = kFused ? 2 : 1;  // 16-byte words of activation per row per chunk
  // The decode table first, at LDS address 0.
  __shared__ __attribute__((aligned(16))) uint8_t dec_tab[kRep ? kRepLutBytes : 512];
  __shared__ __attribute__((aligned(16))) uint8_t enc_lut[kFused ? 8192 : 16];
  __shared__ __attribute__((aligned(16))) float red[kWaves][kVp];

  const int tid = threadIdx.x;
  const auto dec_lut = decode_lut<kRep>(dec_tab, tid & 63);
  const int n0 = blockIdx.x * kR;
  const int chunks = k >> 4;
  // Weight row of block row r: consecutive rows, or (pair.inter > 0) gate
  // rows i0 + r and up rows inter + i0 + r - kR / 2.
  const bool paired = pair.inter > 0;
  constexpr int kHalf = kR / 2;
  auto row_of = [&](int r) -> int {
    if (!paired) return n0 + r;
    const int i = blockIdx.x * kHalf + (r < kHalf ? r : r - kHalf);
    return r < kHalf ? i : pair.inter + i;
  };

  // Raw operands of one 16-byte column chunk: kR weight rows + kM activation rows.
  u32x4 wq[kR];
  u32x4 ar[kM][kActWords];
  // Activation loads go first: their decode then waits only for them while
  // the weight loads are still in flight.
  auto load = [&](int c) {
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      if constexpr (kFused) {
        const u32x4 *x = reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(act) + size_t(m) * k + 16 * c);
        ar[m][0] = x[0];
        ar[m][1] = x[1];
      } else {
        ar[m][0] = reinterpret_cast<const u32x4 *>(static_cast<const uint8_t *>(act) + size_t(m) * k)[c];
      }
    }
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      // Rows past n re-read row n-1; their sums are never stored.
      const int row = min(row_of(r), n - 1);
      // Weights are read once per call: non-temporal (streaming) loads.
      wq[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(weight + size_t(row) * k) + c);
    }
  };
  // In the one-chunk kernel the chunk's loads go out before the LDS set-up
  // and stay in flight across the barrier: the kernel pays one memory round
  // trip before its first products, not two.  The 256-entry decode table is
  // computed, one entry per thread; the fused kinds' 8 KiB encode table is
  // copied from global memory, so its loads are issued first and its LDS
  // stores wait for them alone (global loads return in order).  The chunk
  // load is unconditional (a thread past the last chunk re-reads it and
  // skips its products): a load under a branch makes the wait counts after
  // the branch conservative, and the table stores would wait for the weights
  // too.  In a loop the preloaded registers stay live across the loop and
  // the kernel spills, hence the separate one-chunk kernel; preloading two or
  // three chunks per thread (k up to 12288) measured no faster for code
  // activations and slower fused.
  static_assert(!kOneChunk || !kDynamic, "the one-chunk kernel takes a fixed activation scale");
  u32x4 enc_part[2];
  if constexpr (kFused) {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(kDeviceTables.static_encode);
    enc_part[0] = src[tid];
    enc_part[1] = src[tid + kThreads];
  }
  // The plain table's entry is computed before the chunk loads, the
  // replicated table's after them (each order measured faster for its table).
  uint32_t entry = kRep ? 0u : decode_entry(tid);
  if constexpr (kOneChunk) load(min(tid, chunks - 1));
  if constexpr (kRep) entry = decode_entry(tid);
  fill_decode_table<kRep>(dec_tab, tid, entry);
  if constexpr (kFused) {
    u32x4 *dst = reinterpret_cast<u32x4 *>(enc_lut);
    dst[tid] = enc_part[0];
    dst[tid + kThreads] = enc_part[1];
  }
  // Without this fence the scheduler moves work across the preload and the
  // one-chunk kernels spill.
  if constexpr (kOneChunk) __builtin_amdgcn_sched_barrier(0);
  lds_barrier();

  // Activation scale of each row: the fixed one, or (dynamic) the row's
  // finite amax floored at 1e-12, reduced over the whole row by the block.
  float row_s[kM], row_r[kM];
  if constexpr (kDynamic) {
    __shared__ float amax_red[kM][kThreads / kWave];
    float m_loc[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) m_loc[m] = 0.f;
    for (int c = tid; c < chunks; c += kThreads) {
#pragma unroll
      for (int m = 0; m < kM; ++m) {
        const u32x4 *xp = reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(act) + size_t(m) * k + 16 * c);
        const u32x4 h[2] = {xp[0], xp[1]};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t w = h[i >> 2][i & 3];
          const float v0 = lo_to_float<kInBf16>(w), v1 = hi_to_float<kInBf16>(w);
          if (__builtin_isfinite(v0)) m_loc[m] = fmaxf(m_loc[m], fabsf(v0));
          if (__builtin_isfinite(v1)) m_loc[m] = fmaxf(m_loc[m], fabsf(v1));
        }
      }
    }
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      const float w = wave_max(m_loc[m]);
      if (tid % kWave == 0) amax_red[m][tid / kWave] = w;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      float a = amax_red[m][0];
#pragma unroll
      for (int w = 1; w < kThreads / kWave; ++w) a = fmaxf(a, amax_red[m][w]);
      row_s[m] = fmaxf(a, 1.0e-12f);
      row_r[m] = __builtin_amdgcn_rcpf(row_s[m]);
    }
  } else {
    const float fixed = kFused ? act_scale[0] : 0.f;
    const float rcp = kFused ? __builtin_amdgcn_rcpf(fixed) : 0.f;
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      row_s[m] = fixed;
      row_r[m] = rcp;
    }
  }
  float acc[kR][kM];
#pragma unroll
  for (int r = 0; r < kR; ++r)
#pragma unroll
    for (int m = 0; m < kM; ++m) acc[r][m] = 0.f;

  // Products of the chunk whose operands are in wq / ar.
  auto compute = [&]() {
    uint32_t a[kM][8];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      if constexpr (kFused) {
        u32x4 lo, hi;
        fast_encode_decode16<kInBf16>(ar[m][0], ar[m][1], row_s[m], row_r[m], enc_lut, dec_lut, lo, hi);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[m][i] = lo[i];
          a[m][4 + i] = hi[i];
        }
      } else {
        decode16(dec_lut, ar[m][0], a[m]);
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
  };
  if constexpr (kOneChunk) {
    if (tid < chunks) compute();
  } else {
    for (int c = tid; c < chunks; c += kThreads) {
      load(c);
      compute();
    }
  }

  // Each wavefront sums its partials in registers; the kWaves wavefront
  // totals of each output meet in LDS.
  const int lane = tid % kWave;
  float vals[kVp];
#pragma unroll
  for (int v = 0; v < kVp; ++v) vals[v] = v < kV ? acc[v / kM][v % kM] : 0.f;
  const float wsum = wave_transpose_sum<kVp>(vals, lane);
  constexpr int kGroup = kWave / kVp;  // lanes holding one total
  if (lane % kGroup == 0) red[tid / kWave][lane / kGroup] = wsum;
  __syncthreads();
  const int v = tid;
  float s = 0.f;
  if (v < kV) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += red[w][v];
  }
  if (v < kV) {
    const int r = v / kM, m = v % kM;
    const int row = paired ? min(row_of(r), n - 1) : n0 + r;
    if (row < n) {
      float ts = kFused ? row_s[0] : act_scale[m];
      if constexpr (kFused) {
#pragma unroll
        for (int mm = 1; mm < kM; ++mm)
          if (m == mm) ts = row_s[mm];
      }
      float y = s * ts * cs[row];
      if (bias) y += load_bias(bias, bias_dtype, row);
      if (paired) {
        red[0][v] = half_bits_to_float<true>(float_to_bf16_bits(y));  // the bf16 GEMV output
      } else {
        store_out(out, out_dtype, size_t(m) * n + row, y);
        if (row < conv.channels) conv_epilogue(conv, m, row, y);
      }
    }
  }
  if (paired) {
    // Every wave has read red above (the sums before the barrier); the
    // gate / up pairs meet in red[0] after this one.
    __syncthreads();
    if (v < kHalf * kM) {
      const int r = v / kM, m = v % kM;
      const int i = blockIdx.x * kHalf + r;
      if (i < pair.inter) {
        const float g = red[0][v], u = red[0][v + kHalf * kM];
        const float act = half_bits_to_float<true>(float_to_bf16_bits(g / (1.f + expf(-g)) * u));
        const float qs = pair.qs[0];
        const float q = act * __builtin_amdgcn_rcpf(qs);
        uint32_t code;
        if (__builtin_expect(near_index_boundary(q), 0)) {
          const float x = act / qs;
          code = __builtin_isnan(x) ? uint32_t(kNan) : kDeviceTables.static_encode[__float_as_uint(x) >> 19];
        } else {
          code = kDeviceTables.static_encode[__float_as_uint(q) >> 19];
        }
        pair.codes[size_t(m) * pair.inter + i] = uint8_t(code);
      }
    }
    if (blockIdx.x == 0 && v < kM) pair.row_scale[v] = pair.qs[0];
  }
}

// ------------------------------------------------------------------------
// MFMA-4 GEMV for 2 <= M <= 4 (code activations, k % 16 == 0, 16-byte aligned
// operands).  v_mfma_f32_4x4x4_16b_bf16 runs 16 independent 4 x 4 x 4
// products per wavefront, product b on lanes 4b .. 4b + 3: A row r comes from
// lane 4b + r, B column j from lane 4b + j, and D[r][j] lands in lane 4b + j,
// element r.  Lane 4b + j of wavefront w loads the 16-byte chunks
// b + 16 s + 64 w + 256 p (s = 0..3, pass p) of weight row 4g + j of each
// row group g of the block, and of activation row j: a load instruction
// covers four rows x 256 contiguous bytes (measured on MI355X, one-shot
// blocks over 100 MB: 5.85 TB/s, against 6.0 TB/s for 1 KiB of one row and
// 5.3 TB/s for sixteen rows x 64 bytes), and the four lanes of each product
// hold the same k positions, so A (four weight rows) and B (the activation
// rows, zero past M) feed the MFMA without any data movement.  The MFMA does
// the M products and the k sums; the VALU only decodes (one table lookup per
// code) - against the dot2 kernel's M / 2 products per weight code plus the
// lane reduction of kR x M partials, which bound it at M = 4.  At the end
// each lane holds kR partial sums of its product's 64-code k range; lane
// bits 5 and 4 are summed by permlane swaps that halve the values per lane,
// bits 3 and 2 by DPP rotations (bits 1..0 are the activation row), and the
// four wavefronts meet in LDS.
typedef short s16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4_t c) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4_t, u32x2_t{a0, a1}),
                                                 __builtin_bit_cast(s16x4_t, u32x2_t{b0, b1}), c, 0, 0, 0);
}

// Sum of v over the lanes that share bits 0-1 of the lane index and bits 2-3
// (one 16-lane row): DPP rotations by 8 and 4 within the row.
__device__ __forceinline__ float row_quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  return v;
}

// kPasses: 1..3 passes of 4096 k bytes per block, unrolled (k <= 4096 kPasses),
// or 0 for any k (a loop without prefetch).
// kSrc: code activations (kActCodes, act = uint8 [M, k], act_scale = the
// token scales) or the fused static kinds (kActF16 / kActBf16, act = x [M, k],
// act_scale = the fixed scale [1]): each lane encodes and decodes its own
// activation chunks through the quantise-dequantise table (QdqTable), whose
// 16 KiB copy is requested before the chunk loads, so the table stores wait
// for its loads alone.
template <int kM, int kR, int kPasses, bool kRep, int kSrc>
__global__ __launch_bounds__(kThreads, 2) void gemv_mfma4_kernel(
    const void *act, const float *__restrict__ act_scale, const uint8_t *weight, const float *__restrict__ cs,
    const void *__restrict__ bias, int bias_dtype, void *__restrict__ out, int out_dtype, int n, int k,
    const GemvConv conv) {
  static_assert(kR % 4 == 0 && kR <= 16 && kM >= 1 && kM <= 4, "row groups of four, up to four activation rows");
  static_assert(kSrc == kActCodes || kSrc == kActF16 || kSrc == kActBf16, "codes or a fixed activation scale");
  constexpr bool kFused = kSrc != kActCodes;
  constexpr int kAW = kFused ? 2 : 1;     // 16-byte words of activation per chunk
  constexpr int kG = kR / 4;              // row groups
  constexpr int kWaves = kThreads / kWave;
  constexpr int kPass = 16 * kThreads;    // k bytes per pass of the block
  // The decode table first, at LDS address 0.
  __shared__ __attribute__((aligned(16))) uint8_t dec_tab[kRep ? kRepLutBytes : 512];
  __shared__ __attribute__((aligned(16))) float red[kWaves][kR][4];
  __shared__ __attribute__((aligned(16))) uint16_t qdq[kFused ? 8192 : 8];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const auto dec_lut = decode_lut<kRep>(dec_tab, lane);
  const int b = lane >> 2, j = lane & 3;
  const int n0 = blockIdx.x * kR;
  const int chunks = k >> 4;
  // This lane's weight rows (rows past n re-read row n - 1; never stored) and
  // activation row (rows past M read row M - 1 and are zeroed after the load).
  const uint8_t *wrow[kG];
#pragma unroll
  for (int g = 0; g < kG; ++g) wrow[g] = weight + size_t(min(n0 + 4 * g + j, n - 1)) * k;
  // 16-byte words of the activation row: codes, or x (two words per chunk).
  const u32x4 *arow = reinterpret_cast<const u32x4 *>(static_cast<const uint8_t *>(act) +
                                                      size_t(min(j, kM - 1)) * k * (kFused ? 2 : 1));
  const bool act_lane = j < kM;

  // Operands of one pass: weight codes [group][step s], activation [step s].
  struct Pass {
    u32x4 w[kG][4], a[4][kAW];
  };
  // Chunk of step s in the pass starting at chunk p0; past the last chunk the
  // lane re-reads it and zeroes the codes (code 0 decodes to +0, and both
  // operands are zeroed, so no 0 x Inf can appear).
  auto load = [&](Pass &q, int p0) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = min(p0 + 64 * wave + 16 * s + b, chunks - 1);
#pragma unroll
      for (int h = 0; h < kAW; ++h) q.a[s][h] = arow[kAW * c + h];
    }
#pragma unroll
    for (int g = 0; g < kG; ++g)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int c = min(p0 + 64 * wave + 16 * s + b, chunks - 1);
        q.w[g][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wrow[g]) + c);
      }
  };
  Pass cur;
  constexpr int kQdqWords = kFused ? 8192 * 2 / 16 / kThreads : 1;  // 16-byte table words per thread
  u32x4 qdq_part[kQdqWords];
  if constexpr (kFused) {
#pragma unroll
    for (int i = 0; i < kQdqWords; ++i) qdq_part[i] = reinterpret_cast<const u32x4 *>(kQdqTable.v)[tid + i * kThreads];
  }
  uint32_t entry = kRep ? 0u : decode_entry(tid);  // order as in gemv_kernel
  load(cur, 0);
  if constexpr (kRep) entry = decode_entry(tid);
  fill_decode_table<kRep>(dec_tab, tid, entry);
  if constexpr (kFused) {
#pragma unroll
    for (int i = 0; i < kQdqWords; ++i) reinterpret_cast<u32x4 *>(qdq)[tid + i * kThreads] = qdq_part[i];
  }
  const float fixed = kFused ? act_scale[0] : 0.f;
  const float rcp = kFused ? __builtin_amdgcn_rcpf(fixed) : 0.f;
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();

  f32x4_t acc[kG];
#pragma unroll
  for (int g = 0; g < kG; ++g) acc[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // kTail: chunks past the end (a pass that is not full) become zero codes.
  auto compute = [&](const Pass &q, int p0, auto tail) {
    constexpr bool kTail = decltype(tail)::value;
    bool cv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) cv[s] = !kTail || p0 + 64 * wave + 16 * s + b < chunks;
    if constexpr (kFused) {
      // Step by step (encode the activation chunk, then its products), each
      // step fenced from the next: one step's encode temporaries live at a
      // time, which keeps the kernel near the code kind's register count.
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bool live = act_lane && cv[s];
        uint32_t as[8];
        fast_qdq16<kSrc == kActBf16>(live ? q.a[s][0] : u32x4{0, 0, 0, 0}, live ? q.a[s][1] : u32x4{0, 0, 0, 0},
                                     fixed, rcp, qdq, as);
#pragma unroll
        for (int g = 0; g < kG; ++g) {
          uint32_t p[8];
          decode16(dec_lut, !kTail || cv[s] ? q.w[g][s] : u32x4{0, 0, 0, 0}, p);
#pragma unroll
          for (int d = 0; d < 4; ++d) acc[g] = mfma4(p[2 * d], p[2 * d + 1], as[2 * d], as[2 * d + 1], acc[g]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
    uint32_t ad[4][8];  // activation row j as bf16 pairs, per step s
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // Rows past M and chunks past k take zero codes / zero x (both give +0).
      const bool live = act_lane && cv[s];
      decode16(dec_lut, live ? q.a[s][0] : u32x4{0, 0, 0, 0}, ad[s]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int g = 0; g < kG; ++g) {
        uint32_t p[8];
        decode16(dec_lut, !kTail || cv[s] ? q.w[g][s] : u32x4{0, 0, 0, 0}, p);
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[g] = mfma4(p[2 * d], p[2 * d + 1], ad[s][2 * d], ad[s][2 * d + 1], acc[g]);
      }
  };
  const std::true_type tail;
  const std::false_type no_tail;
  constexpr int kStep = kPass / 16;  // chunks per pass
  auto last = [&](const Pass &q, int p) {  // the last pass may be partial
    if (p + kStep <= chunks) compute(q, p, no_tail);
    else compute(q, p, tail);
  };
  if constexpr (kPasses == 1) {
    last(cur, 0);
  } else if constexpr (kPasses > 0) {
    // kPasses passes, unrolled, so the wait counts stay exact: the next
    // pass's loads are in flight while the current one is decoded and
    // multiplied (two register sets).
    Pass nxt;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      Pass &q = (p & 1) ? nxt : cur;
      if (p + 1 < kPasses) load((p & 1) ? cur : nxt, (p + 1) * kStep);
      // All of the next pass's loads go out before this pass's math (left to
      // itself the scheduler sinks some of them between the MFMAs and then
      // waits for every load at once).
      __builtin_amdgcn_sched_barrier(0);
      if (p + 1 < kPasses) compute(q, p * kStep, no_tail);
      else last(q, p * kStep);
    }
  } else {
    // Any number of passes, one at a time.
    int p0 = 0;
    for (; p0 + kStep < chunks; p0 += kStep) {
      if (p0) load(cur, p0);
      compute(cur, p0, no_tail);
    }
    if (p0) load(cur, p0);
    last(cur, p0);
  }

  // vals[4 g + r] = row 4 g + r of this lane's product, activation row j.
  float vals[kR];
#pragma unroll
  for (int g = 0; g < kG; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r) vals[4 * g + r] = acc[g][r];
  constexpr int kQ = kR / 4;  // values per lane after the two halving levels
#pragma unroll
  for (int i = 0; i < kR / 2; ++i) vals[i] = exchange_add<5>(vals[i], vals[i + kR / 2], lane);
#pragma unroll
  for (int i = 0; i < kQ; ++i) vals[i] = exchange_add<4>(vals[i], vals[i + kQ], lane);
  // Lane 16 q + 4 t + j now holds rows i + kQ q (i < kQ) summed over lane
  // bits 4-5; the rotations add bits 2-3.
#pragma unroll
  for (int i = 0; i < kQ; ++i) vals[i] = row_quad_sum(vals[i]);
  if (((lane >> 2) & 3) == 0) {
#pragma unroll
    for (int i = 0; i < kQ; ++i) red[wave][i + kQ * (lane >> 4)][j] = vals[i];
  }
  __syncthreads();
  if (tid < kR * kM) {
    const int r = tid / kM, m = tid - r * kM;
    const int row = n0 + r;
    if (row < n) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) sum += red[w][r][m];
      float y = sum * (kFused ? fixed : act_scale[m]) * cs[row];
      if (bias) y += load_bias(bias, bias_dtype, row);
      store_out(out, out_dtype, size_t(m) * n + row, y);
      if (row < conv.channels) conv_epilogue(conv, m, row, y);
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
  const bool dyn = act_kind == kActF16Dyn || act_kind == kActBf16Dyn;
  const bool in_bf16 = act_kind == kActBf16 || act_kind == kActBf16Dyn;
  const float fixed = act_kind == kActCodes || dyn ? 1.f : act_scale[0];
  float scale[4] = {fixed, fixed, fixed, fixed};  // activation scale of each row
  if (dyn) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m < m_rows) {
        float amax = 0.f;
        for (int kk = lane; kk < k; kk += kWave) {
          const uint16_t h = static_cast<const uint16_t *>(act)[size_t(m) * k + kk];
          const float xv = in_bf16 ? half_bits_to_float<true>(h) : half_bits_to_float<false>(h);
          if (__builtin_isfinite(xv)) amax = fmaxf(amax, fabsf(xv));
        }
        scale[m] = fmaxf(wave_max(amax), 1.0e-12f);
      }
    }
  }
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
          const float xv = in_bf16 ? half_bits_to_float<true>(h) : half_bits_to_float<false>(h);
          code = static_encode_bits(__float_as_uint(xv / scale[m]));
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
    const float sm = m == 0 ? scale[0] : (m == 1 ? scale[1] : (m == 2 ? scale[2] : scale[3]));
    const float ts = act_kind == kActCodes ? act_scale[m] : sm;
    float y = a * ts * cs[row];
    if (bias) y += load_bias(bias, bias_dtype, row);
    store_out(out, out_dtype, size_t(m) * n + row, y);
  }
}

// ------------------------------------------------------------------------
// MFMA-reduced GEMV (k % 64 == 0).  A block of 8 wavefronts owns 16 weight
// rows; wavefront w streams its share of the 64-byte k-steps.  In one step,
// lane l loads 16 contiguous bytes of row n0 + l%16 at k offset 16*(l/16), so
// a load instruction covers 16 rows x 64 contiguous bytes.  The 16 bytes are
// LUT-decoded to bf16 and used as the B operand of two
// v_mfma_f32_16x16x32_bf16 (bytes 0-7 and 8-15); the A operand holds the
// matching activation values for rows m = l%16 < M (zeros otherwise), read
// from a bf16 copy of the activation decoded once per block into LDS.  The
// MFMA does the k-reduction across lanes, so the VALU work per weight byte is
// just the table decode.  D[m][n] lands in lane n, register m.  The eight
// wavefront partials meet in LDS and one pass applies the epilogue.
constexpr int kMfmaWaves = 8;
constexpr int kMfmaThreads = kMfmaWaves * kWave;
constexpr int kMfmaUnroll = 8;  // 16-byte weight loads in flight per lane
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int kM, int kSrc>
__global__ __launch_bounds__(kMfmaThreads, 1) void gemv_mfma_kernel(
    const void *__restrict__ act, const float *__restrict__ act_scale,
    const uint8_t *__restrict__ weight, const float *__restrict__ cs,
    const void *__restrict__ bias, int bias_dtype, void *__restrict__ out, int out_dtype,
    int n, int k) {
  constexpr bool kFused = kSrc != kActCodes;
  // Static LDS first: the decode table sits at LDS address 0, so a table
  // address is one SDWA shift of the weight byte.
  __shared__ __attribute__((aligned(16))) uint16_t dec_tab[256];
  __shared__ __attribute__((aligned(16))) uint32_t zero_block[8];
  const CompactLut dec_lut{dec_tab};
  __shared__ __attribute__((aligned(16))) float red[kMfmaWaves * 16 * 4];
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t *xs = reinterpret_cast<uint16_t *>(smem);                       // [kM][k] bf16
  uint8_t *enc_lut = smem + size_t(kM) * k * 2;                             // 8 KiB (fused)

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n0 = blockIdx.x * 16;
  const int steps = k >> 6;
  const int s_begin = (steps * wave) / kMfmaWaves, s_end = (steps * (wave + 1)) / kMfmaWaves;
  const uint8_t *wptr = weight + size_t(min(n0 + (lane & 15), n - 1)) * k + ((lane >> 4) << 4);

  // Weight loads go out first and stay in flight through the prologue.
  u32x4 wq[kMfmaUnroll];
#pragma unroll
  for (int u = 0; u < kMfmaUnroll; ++u)
    if (s_begin + u < s_end) wq[u] = *reinterpret_cast<const u32x4 *>(wptr + size_t(s_begin + u) * 64);

  if (tid < 128) reinterpret_cast<uint32_t *>(dec_tab)[tid] = reinterpret_cast<const uint32_t *>(kDeviceTables.decode_bf16)[tid];
  if (tid < 8) zero_block[tid] = 0u;
  if constexpr (kFused) reinterpret_cast<u32x4 *>(enc_lut)[tid] = reinterpret_cast<const u32x4 *>(kDeviceTables.static_encode)[tid];
  lds_barrier();

  // Activation -> bf16 in LDS, once per block.
  {
    const int row_chunks = k >> 4;
    const float s = kFused ? act_scale[0] : 0.f;
    const float r = kFused ? __builtin_amdgcn_rcpf(s) : 0.f;
    for (int c = tid; c < kM * row_chunks; c += kMfmaThreads) {
      const int m = c / row_chunks, kc = c - m * row_chunks;
      u32x4 lo, hi;
      if constexpr (kFused) {
        const u32x4 *x = reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(act) + size_t(m) * k + 16 * kc);
        fast_encode_decode16<kSrc == kActBf16>(x[0], x[1], s, r, enc_lut, dec_lut, lo, hi);
      } else {
        uint32_t p[8];
        decode16(dec_lut, reinterpret_cast<const u32x4 *>(static_cast<const uint8_t *>(act) + size_t(m) * k)[kc], p);
        lo = u32x4{p[0], p[1], p[2], p[3]};
        hi = u32x4{p[4], p[5], p[6], p[7]};
      }
      u32x4 *d = reinterpret_cast<u32x4 *>(xs + size_t(m) * k + 16 * kc);
      d[0] = lo;
      d[1] = hi;
    }
  }
  lds_barrier();

  // A-operand rows m >= kM read a zero block that does not move with k.
  const bool act_lane = (lane & 15) < kM;
  const uint16_t *xa_base = act_lane ? xs + size_t(lane & 15) * k + ((lane >> 4) << 4)
                                     : reinterpret_cast<const uint16_t *>(zero_block);
  const int xa_step = act_lane ? 64 : 0;
  f32x4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  auto step = [&](int s, const u32x4 q) {
    uint32_t p[8];
    decode16(dec_lut, q, p);
    const u32x4 *xa = reinterpret_cast<const u32x4 *>(xa_base + s * xa_step);
    const u32x4 a0 = xa[0], a1 = xa[1];
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a0),
                                                   __builtin_bit_cast(bf16x8_t, u32x4{p[0], p[1], p[2], p[3]}),
                                                   acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a1),
                                                   __builtin_bit_cast(bf16x8_t, u32x4{p[4], p[5], p[6], p[7]}),
                                                   acc1, 0, 0, 0);
  };
  int s0 = s_begin;
  for (; s0 + kMfmaUnroll <= s_end; s0 += kMfmaUnroll) {
#pragma unroll
    for (int u = 0; u < kMfmaUnroll; ++u) {
      const u32x4 q = wq[u];
      if (s0 + kMfmaUnroll + u < s_end)
        wq[u] = *reinterpret_cast<const u32x4 *>(wptr + size_t(s0 + kMfmaUnroll + u) * 64);
      step(s0 + u, q);
    }
  }
#pragma unroll
  for (int u = 0; u < kMfmaUnroll; ++u)
    if (s0 + u < s_end) step(s0 + u, wq[u]);

  if (lane < 16) {
    float *dst = red + (wave * 16 + lane) * 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[r] = acc0[r] + acc1[r];
  }
  lds_barrier();
  if (tid < 64) {
    const int m = tid >> 4, nl = tid & 15;
    const int row = n0 + nl;
    if (m < kM && row < n) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kMfmaWaves; ++w) sum += red[(w * 16 + nl) * 4 + m];
      const float ts = kFused ? act_scale[0] : act_scale[m];
      float y = sum * ts * cs[row];
      if (bias) y += load_bias(bias, bias_dtype, row);
      store_out(out, out_dtype, size_t(m) * n + row, y);
    }
  }
}

template <int kM, int kSrc>
int launch_mfma(const LinearArgs &a) {
  const size_t smem = size_t(kM) * size_t(a.k) * 2 + (kSrc != kActCodes ? 8192 : 0);
  if (const int st = reserve_dynamic_lds(reinterpret_cast<const void *>(&gemv_mfma_kernel<kM, kSrc>), smem,
                                         "soft_hif8 GEMV"))
    return st;
  gemv_mfma_kernel<kM, kSrc><<<dim3(unsigned((a.n + 15) / 16)), kMfmaThreads, smem, a.stream>>>(
      a.act, a.act_scale, a.weight, a.channel_scale, a.bias, a.bias_dtype, a.out, a.out_dtype, int(a.n), int(a.k));
  return HIF8_OK;
}

template <int kM>
int launch_mfma_src(const LinearArgs &a) {
  switch (a.act_kind) {
    case kActCodes: return launch_mfma<kM, kActCodes>(a);
    case kActF16: return launch_mfma<kM, kActF16>(a);
    default: return launch_mfma<kM, kActBf16>(a);
  }
}

// LDS bytes the MFMA GEMV needs, or 0 when the shape does not fit it.
size_t mfma_gemv_smem(const LinearArgs &a) {
  if (a.k % 64 || !aligned(a.weight, 16) || !aligned(a.act, 16)) return 0;
  const size_t smem = 512 + 32 + 2048 + size_t(a.m) * size_t(a.k) * 2 + (a.act_kind != kActCodes ? 8192 : 0);
  return smem <= 160 * 1024 ? smem : 0;
}

enum GemvKind { kGemvDot2, kGemvMfma4, kGemvSimple, kGemvMfma16 };

struct GemvPlan {
  GemvKind kind;
  int rows;        // weight rows per block
  bool one_chunk;  // k <= 16 * 256: one 16-byte chunk (dot2) or one pass (MFMA-4) per thread
  unsigned grid;
  unsigned threads;
  bool rep;        // replicated (conflict-free) decode table
};

template <int kM, int kR, bool kRep>
void dispatch_src(const LinearArgs &a, dim3 grid) {
  const int n = int(a.n), k = int(a.k);
#define HIF8_DOT2_LAUNCH(SRC, ONE, REP)                                                                    \
  gemv_kernel<kM, kR, SRC, ONE, REP><<<grid, kThreads, 0, a.stream>>>(                                   \
      a.act, a.act_scale, a.weight, a.channel_scale, a.bias, a.bias_dtype, a.out, a.out_dtype, n, k, a.pair, a.conv)
  const bool one = k <= 16 * kThreads;
  switch (a.act_kind) {
    case kActCodes:
      if (one) HIF8_DOT2_LAUNCH(kActCodes, true, kRep);
      else HIF8_DOT2_LAUNCH(kActCodes, false, kRep);
      break;
    case kActF16:
      if (one) HIF8_DOT2_LAUNCH(kActF16, true, kRep);
      else HIF8_DOT2_LAUNCH(kActF16, false, kRep);
      break;
    case kActBf16:
      if (one) HIF8_DOT2_LAUNCH(kActBf16, true, kRep);
      else HIF8_DOT2_LAUNCH(kActBf16, false, kRep);
      break;
    case kActF16Dyn: HIF8_DOT2_LAUNCH(kActF16Dyn, false, kRep); break;
    default: HIF8_DOT2_LAUNCH(kActBf16Dyn, false, kRep); break;
  }
#undef HIF8_DOT2_LAUNCH
}

template <int kR>
void dispatch_m(const LinearArgs &a, const GemvPlan &p) {
  const dim3 grid(p.grid);
  if (p.rep) {
    switch (a.m) {
      case 1: dispatch_src<1, kR, true>(a, grid); break;
      case 2: dispatch_src<2, kR, true>(a, grid); break;
      case 3: dispatch_src<3, kR, true>(a, grid); break;
      default: dispatch_src<4, kR, true>(a, grid); break;
    }
    return;
  }
  switch (a.m) {
    case 1: dispatch_src<1, kR, false>(a, grid); break;
    case 2: dispatch_src<2, kR, false>(a, grid); break;
    case 3: dispatch_src<3, kR, false>(a, grid); break;
    default: dispatch_src<4, kR, false>(a, grid); break;
  }
}

// Kernel selection knobs, read once: HIF8_GEMV_KERNEL=d forces the dot2 VALU
// kernel for every M (default: the MFMA-4 kernel for code activations at
// M = 4, and M = 3 over wide weights), =4 the MFMA-4 kernel for every M >= 2,
// =m the experimental 16x16x32 MFMA kernel; HIF8_GEMV_ROWS=4|8|12|16
// forces the rows per block (12: M = 1 or the MFMA-4 kernel);
// HIF8_GEMV_LUT=r|c forces the replicated or the compact decode table.  Measured on
// MI355X (gate_up 24576x4096, M=1): the dot2 kernel with 8 rows per block
// 20.0 us; the 16x16x32 MFMA kernel 29.3 us (its 16-rows x 64-byte load
// pattern alone reads ~12 % slower than 1 KiB-contiguous rows); a persistent
// double-buffered variant 24 us (2 blocks/CU keep too few bytes in flight).
struct GemvKnobs {
  char kernel = 'v';
  int rows = 0;
  char lut = 0;  // 'r' replicated, 'c' compact, else by grid size
  GemvKnobs() {
    if (const char *v = getenv("HIF8_GEMV_KERNEL")) kernel = v[0];
    if (const char *v = getenv("HIF8_GEMV_ROWS")) rows = atoi(v);
    if (const char *v = getenv("HIF8_GEMV_LUT")) lut = v[0];
  }
};

GemvPlan plan_gemv(int64_t m, int64_t n, int64_t k, int act_kind, bool vec) {
  static const GemvKnobs knobs;
  const bool dynamic = act_kind == kActF16Dyn || act_kind == kActBf16Dyn;
  GemvPlan p{};
  p.one_chunk = k <= 16 * kThreads;
  p.threads = kThreads;
  if (!vec) {
    p.kind = kGemvSimple;
    p.rows = 1;
    p.threads = kWave;
    p.grid = unsigned(n);
    return p;
  }
  const bool wide = n >= 16384;
  if (knobs.kernel == 'm' && !dynamic && k % 64 == 0) {
    p.kind = kGemvMfma16;
    p.rows = 16;
    p.threads = kMfmaThreads;
  } else if (knobs.kernel != 'd' && (act_kind == kActCodes || act_kind == kActF16 || act_kind == kActBf16) &&
             ((k <= 16 * kThreads && (m == 4 || (m == 3 && wide))) || (knobs.kernel == '4' && m >= 2))) {
    // Code activations, four rows (three over wide weights), k <= 4096: the
    // MFMA does the products.  Measured on MI355X (graphs of 20 launches over
    // >= 768 MB of weights), against the dot2 kernel: M = 4 gate_up 20.3 vs
    // 23.2 us, q / o 6.4 vs 6.8, k+v 4.95 vs 5.1; M = 3 gate_up 20.2 vs 22.1;
    // but M = 2, the narrow M = 3 shapes (q M = 2 6.0 vs 7.1) and the
    // multi-pass down projection (k = 12288, M = 4: 14.8 vs 14.3, also with
    // the next pass prefetched) are faster on dot2.
    p.kind = kGemvMfma4;
    const int r = knobs.rows;
    p.rows = r == 4 || r == 8 || r == 12 || r == 16 ? r : (wide ? 16 : 8);
  } else {
    // 8 rows per block; over wide weights (N >= 16384) M = 4 streams faster
    // with 16 (gate_up 24576 x 4096: 24.8 vs 25.7-26.5 us on MI355X) and
    // M = 1 with 12, 2048 blocks (17.4-17.6 vs 17.8 us; 6 rows 17.6-18.3).
    // M = 1 takes 12 rows from N = 8192 on: the one-launch fused static kind
    // over 12288 x 4096 runs 12.3 vs 13.9 us (the code GEMV 11.09 vs 11.07).
    // q/o/k-v and down are fastest with 8.
    p.kind = kGemvDot2;
    const int r = knobs.rows ? knobs.rows : (wide && m == 4 ? 16 : m == 1 && n >= 8192 ? 12 : 8);
    p.rows = r >= 16 ? 16 : r == 12 && m == 1 ? 12 : r >= 8 ? 8 : 4;
  }
  p.grid = unsigned((n + p.rows - 1) / p.rows);
  // The replicated table for grids of one round, except the single-row k
  // loop (down 4096 x 12288 at M = 1: 11.07 vs 10.85 us on MI355X).
  // The fused static kinds of the MFMA-4 kernel hold a 16 KiB
  // quantise-dequantise table, with which the 64 KiB replicated table would
  // no longer leave room for two blocks per CU: they take the plain table.
  const bool mfma4_fused = p.kind == kGemvMfma4 && act_kind != kActCodes;
  p.rep = !mfma4_fused && (knobs.lut == 'r' || (knobs.lut != 'c' && p.grid <= kRepMaxBlocks &&
                                                 !(m == 1 && p.kind == kGemvDot2 && !p.one_chunk)));
  return p;
}

// Passes of 4096 k bytes the MFMA-4 kernel unrolls for this k (0: a loop).
int mfma4_passes(int64_t k) {
  const int64_t passes = (k + 16 * kThreads - 1) / (16 * kThreads);
  return passes <= 3 ? int(passes) : 0;
}

template <int kM, int kR, bool kRep, int kSrc>
void launch_mfma4_t(const LinearArgs &a, const GemvPlan &p) {
#define HIF8_MFMA4_LAUNCH(P)                                                                              \
  gemv_mfma4_kernel<kM, kR, P, kRep, kSrc><<<p.grid, kThreads, 0, a.stream>>>(                          \
      a.act, a.act_scale, a.weight, a.channel_scale, a.bias, a.bias_dtype, a.out, a.out_dtype, int(a.n), int(a.k), \
      a.conv)
  // Two register sets of more than eight rows exceed the register file.
  constexpr bool kTwoSets = kR <= 8;
  switch (mfma4_passes(a.k)) {
    case 1: HIF8_MFMA4_LAUNCH(1); break;
    case 2: if constexpr (kTwoSets) { HIF8_MFMA4_LAUNCH(2); } else { HIF8_MFMA4_LAUNCH(0); } break;
    case 3: if constexpr (kTwoSets) { HIF8_MFMA4_LAUNCH(3); } else { HIF8_MFMA4_LAUNCH(0); } break;
    default: HIF8_MFMA4_LAUNCH(0); break;
  }
#undef HIF8_MFMA4_LAUNCH
}

// The fused kinds always take the plain table (see plan_gemv).
template <int kM, int kR, int kSrc>
void launch_mfma4_s(const LinearArgs &a, const GemvPlan &p) {
  if (kSrc == kActCodes && p.rep) launch_mfma4_t<kM, kR, kSrc == kActCodes, kSrc>(a, p);
  else launch_mfma4_t<kM, kR, false, kSrc>(a, p);
}

template <int kM, int kR>
void launch_mfma4(const LinearArgs &a, const GemvPlan &p) {
  switch (a.act_kind) {
    case kActCodes: launch_mfma4_s<kM, kR, kActCodes>(a, p); break;
    case kActF16: launch_mfma4_s<kM, kR, kActF16>(a, p); break;
    default: launch_mfma4_s<kM, kR, kActBf16>(a, p); break;
  }
}

template <int kR>
void launch_mfma4_m(const LinearArgs &a, const GemvPlan &p) {
  switch (a.m) {
    case 2: launch_mfma4<2, kR>(a, p); break;
    case 3: launch_mfma4<3, kR>(a, p); break;
    default: launch_mfma4<4, kR>(a, p); break;
  }
}

__global__ __launch_bounds__(256) void conv_rows_kernel(const GemvConv conv, const uint16_t *__restrict__ y,
                                                        int64_t ld, int m_rows) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= m_rows * conv.channels) return;
  const int m = idx / conv.channels, c = idx - m * conv.channels;
  conv_epilogue(conv, m, c, half_bits_to_float<true>(y[size_t(m) * ld + c]));
}

}  // namespace

int launch_conv_rows(const GemvConv &conv, const uint16_t *y, int64_t ld, int64_t m, hipStream_t stream) {
  if (conv.channels <= 0 || conv.kw < 2 || conv.kw > 4 || m <= 0 || ld < conv.channels ||
      m * conv.channels > 0x7FFFFFFFll || !y || !conv.weight || !conv.state || !conv.out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "conv epilogue: invalid arguments");
  const int64_t items = m * conv.channels;
  conv_rows_kernel<<<unsigned((items + 255) / 256), 256, 0, stream>>>(conv, y, ld, int(m));
  return check_launch("conv epilogue");
}

int launch_gemv(const LinearArgs &a) {
  if (a.m < 1 || a.m > 4) return fail(HIF8_ERR_UNSUPPORTED, "GEMV kernel handles 1 <= M <= 4, got %lld", (long long)a.m);
  const bool vec = a.k % 16 == 0 && aligned(a.weight, 16) && aligned(a.act, 16);
  const GemvPlan p = plan_gemv(a.m, a.n, a.k, a.act_kind, vec);
  if (a.pair.inter > 0 && (p.kind != kGemvDot2 || a.n != 2 * int64_t(a.pair.inter) || a.bias))
    return fail(HIF8_ERR_UNSUPPORTED, "gate_up + SiLU-mul GEMV: the plan for M=%lld N=%lld K=%lld is not the dot2 kernel",
                (long long)a.m, (long long)a.n, (long long)a.k);
  if (a.conv.channels > 0 && ((p.kind != kGemvDot2 && p.kind != kGemvMfma4) || a.pair.inter > 0 ||
                              a.out_dtype != HIF8_DTYPE_BF16 || a.conv.channels > a.n || a.conv.kw < 2 ||
                              a.conv.kw > 4 || !a.conv.weight || !a.conv.state || !a.conv.out))
    return fail(HIF8_ERR_UNSUPPORTED, "conv-epilogue GEMV: the plan for M=%lld N=%lld K=%lld has no conv epilogue",
                (long long)a.m, (long long)a.n, (long long)a.k);
  switch (p.kind) {
    case kGemvSimple:
      gemv_simple_kernel<<<p.grid, kWave, 0, a.stream>>>(a.act, a.act_kind, a.act_scale, a.weight, a.channel_scale,
                                                         a.bias, a.bias_dtype, a.out, a.out_dtype, int(a.m),
                                                         int(a.n), int(a.k));
      break;
    case kGemvMfma16: {
      int st = HIF8_OK;
      if (!mfma_gemv_smem(a)) return fail(HIF8_ERR_UNSUPPORTED, "soft_hif8 GEMV: the MFMA kernel cannot take this shape");
      switch (a.m) {
        case 1: st = launch_mfma_src<1>(a); break;
        case 2: st = launch_mfma_src<2>(a); break;
        case 3: st = launch_mfma_src<3>(a); break;
        default: st = launch_mfma_src<4>(a); break;
      }
      if (st) return st;
      break;
    }
    case kGemvMfma4:
      switch (p.rows) {
        case 4: launch_mfma4_m<4>(a, p); break;
        case 8: launch_mfma4_m<8>(a, p); break;
        case 12: launch_mfma4_m<12>(a, p); break;
        default: launch_mfma4_m<16>(a, p); break;
      }
      break;
    default:
      if (p.rows >= 16) dispatch_m<16>(a, p);
      else if (p.rows == 12 && p.rep) dispatch_src<1, 12, true>(a, dim3(p.grid));
      else if (p.rows == 12) dispatch_src<1, 12, false>(a, dim3(p.grid));
      else if (p.rows >= 8) dispatch_m<8>(a, p);
      else dispatch_m<4>(a, p);
      break;
  }
  return check_launch("soft_hif8 GEMV");
}

int describe_gemv(int64_t m, int64_t n, int64_t k, int act_kind, char *name, size_t name_len, int64_t *grid) {
  const GemvPlan p = plan_gemv(m, n, k, act_kind, k % 16 == 0);
  if (grid) *grid = p.grid;
  if (name && name_len) {
    switch (p.kind) {
      case kGemvSimple: snprintf(name, name_len, "gemv_simple_kernel"); break;
      case kGemvMfma16: snprintf(name, name_len, "gemv_mfma_kernel<%lld, %d>", (long long)m, act_kind); break;
      case kGemvMfma4:
        snprintf(name, name_len, "gemv_mfma4_kernel<%lld, %d, %d, %s, %d>", (long long)m, p.rows,
                 p.rows > 8 && mfma4_passes(k) > 1 ? 0 : mfma4_passes(k), p.rep ? "true" : "false", act_kind);
        break;
      default: {
        const bool dyn = act_kind == kActF16Dyn || act_kind == kActBf16Dyn;
        snprintf(name, name_len, "gemv_kernel<%lld, %d, %d, %s, %s>", (long long)m, p.rows, act_kind,
                 p.one_chunk && !dyn ? "true" : "false", p.rep ? "true" : "false");
      }
    }
  }
  return HIF8_OK;
}

}  // namespace hif8
