// Multi-token paged attention over HiF8 pages for gfx950: prefill and
// chunked prefill (several query tokens per request, right-aligned causal
// mask), decoding the cache pages inside the kernel.
//
// Contract (kv_cache.py:314-372 with query_lens; the reference's TND call of
// npu_fused_infer_attention_score, kv_runtime.py:1470-1563, sparse_mode=3):
// request b owns query rows query_start_loc[b] .. query_start_loc[b + 1] - 1
// and seq_lens[b] cached tokens (this step's tokens included); its query row i
// sits at position seq_lens[b] - q_len + i and, when causal, sees keys
// 0 .. that position.  K and V rows are decoded to dtype(dec(c) * s_row), the
// query dtype (kv_cache.py:355-356), and query head hq attends KV head
// hq / (Hq / Hkv).  A row that sees no key gets zeros.
//
// Work split.  A workgroup (4 wavefronts) owns one (request, KV head, query
// tile of 64 / G tokens, key split): its 64 rows are the (token, query head)
// pairs of the tile, 16 per wavefront, so the G query heads of a KV head
// share every decoded K/V tile.  It walks its key range in 64-key tiles:
//   * all 256 threads load the tile's raw K and V rows (16 bytes per load,
//     rows found through the block table, any block size), decode them with
//     an fp32 table in LDS, multiply by the row's scale, round to the query
//     dtype and store K as [key][D] and V transposed as [D][key] in LDS
//     (16-byte granules XOR-swizzled so the fragment reads spread over banks);
//   * each wavefront computes S^T = K Q^T on v_mfma_f32_16x16x32 (A = 16 keys
//     x 32 dims from LDS, B = its 16 query rows, held in VGPRs for the whole
//     loop), applies the causal / length mask and an online softmax in FP32
//     (base 2), and accumulates O^T += V^T P^T on the same MFMA, P rounded to
//     the query dtype (the reference's probs.to(query.dtype));
//   * the next tile's raw rows are loaded while the current one computes.
// The S^T accumulators leave lane (g, n) holding keys 4g + e and 16 + 4g + e
// of query row n, which are the k-slots 8g + e of the P^T operand of the
// 32-key step; V^T is stored in that key order, so P needs no data movement.
//
// With several key splits per query tile the partial (O, max, sum) go to the
// caller's workspace and a second kernel merges them.  Shapes outside the
// MFMA kernel's set (head size not 64/128/256, Dv != D, G not dividing 16)
// run a one-wavefront-per-(row, head) kernel.
#include <stddef.h>
#include <stdlib.h>

#include <algorithm>

#include "hif8_common.h"

namespace hif8 {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kPThreads = 256;  // four wavefronts
constexpr int kPRows = 64;      // (token, head) rows per workgroup, 16 per wavefront
constexpr int kKT = 64;         // keys per tile
constexpr int kTargetBlocks = 512;
constexpr int kMinSplitTiles = 2;
constexpr int kIThreads = 512;  // tile-image kernel: eight wavefronts
constexpr int kIWaves = kIThreads / 64;
constexpr int kIRows = 128;     // its (token, head) rows per workgroup
constexpr int kITargetBlocks = 256;

// Bytes of one decoded 64-key tile image: K rows [64][D], V^T rows [D][64]
// (16-bit values, swizzled as in LDS), 64 fp32 logit biases, padded to 1 KiB.
constexpr uint32_t img_bytes(int d) { return (uint32_t(4 * kKT * d + 4 * kKT) + 1023u) / 1024u * 1024u; }

struct PrefillParams {
  const void *query;              // [total_q, Hq, D]
  const uint8_t *key_cache;       // [num_blocks, block_size, Hkv, D + 4]
  const uint8_t *value_cache;     // [num_blocks, block_size, Hkv, Dv + 4]
  const void *block_table;        // [batch, bt_stride] int32 or int64
  const int32_t *query_start_loc; // [batch + 1]
  const int32_t *seq_lens;        // [batch]
  void *out;                      // [total_q, Hq, Dv]
  float *part_o;                  // [items, num_splits, kPRows, Dv]
  float *part_ml;                 // [items, num_splits, kPRows, 2]
  int64_t bt_stride;
  int64_t num_blocks;
  int block_size, log2_block_size, hkv, hq, group, log2_group, d, dv;  // log2_block_size -1: not a power of two
  int tokens_per_tile, q_tiles, num_splits, split_tiles, batch, max_len, causal;
  int total_q;                    // rows of query / out; rows at or past it are never touched
  float scale_log2;               // softmax scale * log2(e)
  uint8_t *img;                   // decoded tile images [slots][hkv][img_tiles] (tile-image path)
  int img_tiles;                  // 64-key tiles per (request, KV head) in img
  int slots;                      // image slots (0: no request takes the tile-image path)
  int long_rows;                  // a request is long when its (token, head) rows exceed this
};

// Requests whose query covers more than p.long_rows (token, head) rows take
// the tile-image path when one of the p.slots image slots is theirs: slot s
// belongs to the s-th long request in request order, so short requests in
// the same batch (decode rows of a chunked-prefill step) neither get images
// nor cost image bytes.  Every wavefront of a workgroup evaluates these
// itself from query_start_loc; the results are uniform.
__device__ __forceinline__ bool request_is_long(const PrefillParams &p, int b) {
  const int q_begin = max(p.query_start_loc[b], 0);
  const int ql = min(p.query_start_loc[b + 1], p.total_q) - q_begin;
  return ql > 0 && int64_t(ql) * p.group > int64_t(p.long_rows);
}

// Long requests among 0 .. b - 1 (64 requests per round of the wavefront).
__device__ int long_requests_before(const PrefillParams &p, int b) {
  const int lane = threadIdx.x & 63;
  int count = 0;
  for (int base = 0; base < b; base += 64) {
    const int i = base + lane;
    count += __popcll(__ballot(i < b && request_is_long(p, i)));
  }
  return count;
}

// True when request b runs on the tile-image path.
__device__ __forceinline__ bool request_has_images(const PrefillParams &p, int b) {
  return p.slots > 0 && request_is_long(p, b) && long_requests_before(p, b) < p.slots;
}

// The request holding image slot s, or -1 when fewer requests are long.
__device__ int request_of_slot(const PrefillParams &p, int s) {
  const int lane = threadIdx.x & 63;
  int seen = 0;
  for (int base = 0; base < p.batch; base += 64) {
    const int i = base + lane;
    const bool lg = i < p.batch && request_is_long(p, i);
    const uint64_t mask = __ballot(lg);
    const int c = __popcll(mask);
    if (seen + c > s) {  // the (s - seen)-th long request of this round
      const int rank = __popcll(mask & ((uint64_t(1) << lane) - 1));
      const uint64_t hit = __ballot(lg && rank == s - seen);
      return base + __ffsll(static_cast<unsigned long long>(hit)) - 1;
    }
    seen += c;
  }
  return -1;
}

template <bool kBf16>
__device__ __forceinline__ f32x4_t mfma16(u32x4 a, u32x4 b, f32x4_t c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// Two fp32 values rounded to nearest-even into the MFMA operand dtype, lo in
// the low half (bf16: one v_cvt_pk_bf16_f32 for the pair).
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (kBf16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
  return uint32_t(float_to_f16_bits(lo)) | (uint32_t(float_to_f16_bits(hi)) << 16);
}

// Granule swizzle of K row `key` (16-byte granules of kD bf16 values).  The
// in-kernel path, whose threads write four keys 4 kq + j of a column
// together, folds key >> 4 in so those 16 rows hit 16 bank groups; tile
// images (written to global memory, copied into LDS verbatim) use key & 15
// alone, which leaves the 16 rows one fragment read touches conflict-free
// and makes the swizzle the same for the four 16-key blocks, so a fragment
// address is one of four per-lane bases plus an immediate.
template <int kD, bool kImg>
__device__ __forceinline__ int k_swizzle(int key) {
  constexpr int kKGran = kD / 8;
  constexpr int kKSwz = (kKGran < 16 ? kKGran : 16) - 1;
  return kImg ? key & kKSwz : (key ^ (key >> 4)) & kKSwz;
}

__device__ __forceinline__ int clamp_len(int len, int max_len) {
  return len < 0 ? 0 : (len > max_len ? max_len : len);
}

// Position of key k (0..63) of a tile in the V^T rows: within each 32-key
// half, keys 4g + e sit at 8g + e and keys 16 + 4g + e at 8g + 4 + e.
__device__ __forceinline__ int vt_pos(int k) {
  const int half = k & 32, kk = k & 31;
  return half + (kk < 16 ? 8 * (kk >> 2) + (kk & 3) : 8 * ((kk - 16) >> 2) + 4 + (kk & 3));
}

// Decodes one 64-key tile from the raw rows a thread holds (thread (kq, dc):
// 16-byte chunk dc of keys kq * kD / 64 + j; bit j of `ok` says the key is
// present) into K rows [64][kD] and V^T rows [kD][64] in P^T key order, both
// granule-swizzled, and a per-key logit bias; absent keys become zeros and a
// -inf bias.  The destinations are LDS or a tile image in global memory with
// the same layout.
template <int kD, bool kBf16, bool kImg>
__device__ __forceinline__ void decode_tile(const float *dec, const u32x4 (&kraw)[kD / 64],
                                            const u32x4 (&vraw)[kD / 64], const float (&kscl)[kD / 64],
                                            const float (&vscl)[kD / 64], uint32_t ok, int kq, int dc,
                                            uint16_t *ks, uint16_t *vt, float *kbias) {
  constexpr int kKPT = kD / 64;
#pragma unroll
  for (int j = 0; j < kKPT; ++j) {
    const int kt = kq * kKPT + j;  // key within the tile
    const bool kok = (ok >> j) & 1u;
    const float ksc = kok ? kscl[j] : 0.f;
    uint32_t kw[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) kw[w] = kok ? kraw[j][w] : 0u;
    uint32_t kp[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      kp[2 * w] = pack2<kBf16>(dec[kw[w] & 0xFFu] * ksc, dec[(kw[w] >> 8) & 0xFFu] * ksc);
      kp[2 * w + 1] = pack2<kBf16>(dec[(kw[w] >> 16) & 0xFFu] * ksc, dec[kw[w] >> 24] * ksc);
    }
    const int sw = k_swizzle<kD, kImg>(kt);
    uint16_t *krow = ks + kt * kD;
    *reinterpret_cast<u32x4 *>(krow + 8 * ((2 * dc) ^ sw)) = u32x4{kp[0], kp[1], kp[2], kp[3]};
    *reinterpret_cast<u32x4 *>(krow + 8 * ((2 * dc + 1) ^ sw)) = u32x4{kp[4], kp[5], kp[6], kp[7]};
    if (dc == 0) kbias[kt] = kok ? 0.f : -__builtin_inff();
  }
  // V transposed: dim 16 dc + i', kKPT consecutive keys at consecutive
  // positions.  Odd chunks walk their dims in the order i ^ 1, so the four
  // rows one store instruction writes alternate between the two bank halves.
  {
    const int pos = vt_pos(kq * kKPT);
    float vsc[kKPT];
    uint32_t vw[kKPT][4];
#pragma unroll
    for (int j = 0; j < kKPT; ++j) {
      const bool vok = (ok >> j) & 1u;
      vsc[j] = vok ? vscl[j] : 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) vw[j][w] = vok ? vraw[j][w] : 0u;
    }
    const int flip = dc & 1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int ii = i ^ flip;          // same 4-byte word as i
      const int dim = 16 * dc + ii;
      const int sh = 8 * (ii & 3);
      float v[kKPT];
#pragma unroll
      for (int j = 0; j < kKPT; ++j) v[j] = dec[(vw[j][i >> 2] >> sh) & 0xFFu] * vsc[j];
      const int gran = (pos >> 3) ^ (dim & 7);
      uint16_t *dst = vt + dim * kKT + 8 * gran + (pos & 7);
      if constexpr (kKPT == 4) {
        *reinterpret_cast<u32x2 *>(dst) = u32x2{pack2<kBf16>(v[0], v[1]), pack2<kBf16>(v[2], v[3])};
      } else if constexpr (kKPT == 2) {
        *reinterpret_cast<uint32_t *>(dst) = pack2<kBf16>(v[0], v[1]);
      } else {
        *dst = float_to_half_bits<kBf16>(v[0]);
      }
    }
  }}

// One 64-key tile of a wavefront's kRB blocks of 16 query rows, K ([key][D])
// and V^T ([D][key] in P^T key order) in LDS with the granule swizzles above:
// S^T = K Q^T, the causal / length mask (keys at or past lim[rb]) and the
// per-key bias, the online softmax update of (m, l) in base 2, and
// O^T += V^T P^T with P rounded to the query dtype.  Each K or V^T fragment
// read from LDS feeds the MFMAs of all kRB row blocks.
// Log2 headroom of the lazily updated softmax reference (see tile_math).
constexpr float kLazyMax = 8.f;

// full (wave-uniform): every row of the wavefront sees every key of the tile
// (keys k0 .. k0 + 63 below each lim), so the per-key mask is skipped.
template <int kD, bool kBf16, int kRB, bool kImg>
__device__ __forceinline__ void tile_math(const uint16_t *ks, const uint16_t *vt, const float *kbias,
                                          const u32x4 (&qf)[kRB][kD / 32], int k0, const int (&lim)[kRB],
                                          float scale_log2, int n, int g, float (&m)[kRB], float (&l)[kRB],
                                          f32x4_t (&oacc)[kRB][kD / 16], bool full = false) {
  constexpr int kQSteps = kD / 32;
  constexpr int kDB = kD / 16;
  // S^T = K Q^T: four 16-key blocks.  Lane (g, n) reads granule 4 i + g of
  // key 16 kb + n.  Image layout: the swizzle n' = n & 15 (or & 7) touches
  // granule bits 0-3 only, so granule (4 i + g) ^ n' = 16 (i >> 2) +
  // ((4 (i & 3) + g) ^ n'): four per-lane bases, the rest immediates.
  constexpr int kBases = kQSteps < 4 ? kQSteps : 4;
  const uint16_t *kbase[kBases];
#pragma unroll
  for (int j = 0; j < kBases; ++j) kbase[j] = ks + n * kD + 8 * ((4 * j + g) ^ k_swizzle<kD, true>(n));
  f32x4_t sacc[kRB][4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) sacc[rb][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int key = 16 * kb + n;
    const int sw = k_swizzle<kD, kImg>(key);
    const uint16_t *krow = ks + key * kD;
#pragma unroll
    for (int i = 0; i < kQSteps; ++i) {
      const uint16_t *src = kImg ? kbase[i & 3] + 16 * kb * kD + 128 * (i >> 2) : krow + 8 * ((4 * i + g) ^ sw);
      const u32x4 a = *reinterpret_cast<const u32x4 *>(src);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) sacc[rb][kb] = mfma16<kBf16>(a, qf[rb][i], sacc[rb][kb]);
    }
  }
  // Mask and online softmax (base 2): lane (g, n) holds keys 16 kb + 4 g + e of row n.
  u32x4 pf[kRB][2];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    float x[16];
    float tmax = -__builtin_inff();
    if (full) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const f32x4_t bias = *reinterpret_cast<const f32x4_t *>(kbias + 16 * kb + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[4 * kb + e] = sacc[rb][kb][e] * scale_log2 + bias[e];
          tmax = fmaxf(tmax, x[4 * kb + e]);
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const f32x4_t bias = *reinterpret_cast<const f32x4_t *>(kbias + 16 * kb + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = k0 + 16 * kb + 4 * g + e;
          const float v = sacc[rb][kb][e] * scale_log2 + bias[e];
          x[4 * kb + e] = key < lim[rb] ? v : -__builtin_inff();
          tmax = fmaxf(tmax, x[4 * kb + e]);
        }
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    // m is the reference the row's weights, l and O are taken against; it
    // moves (and l, O are rescaled) only when the row's max exceeds it by
    // more than kLazyMax, so every weight stays below 2^kLazyMax and most
    // tiles skip the rescale (rows start at -inf, where O and l are still 0).
    const bool grow = tmax > m[rb] + kLazyMax;
    if (__any(grow)) {
      const float m_next = grow ? fmaxf(m[rb], tmax) : m[rb];
      if (!__all(!grow || m[rb] == -__builtin_inff())) {
        const float alpha = __builtin_amdgcn_exp2f(m[rb] - (m_next == -__builtin_inff() ? 0.f : m_next));
        l[rb] *= alpha;
#pragma unroll
        for (int db = 0; db < kDB; ++db) oacc[rb][db] *= alpha;
      }
      m[rb] = m_next;
    }
    const float m_use = m[rb] == -__builtin_inff() ? 0.f : m[rb];
    float pw[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) pw[e] = __builtin_amdgcn_exp2f(x[e] - m_use);
    float psum = pw[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) psum += pw[e];
    l[rb] += psum;
    // P^T operands of the two 32-key steps.
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float *a = pw + 8 * s;      // keys 32 s + 4 g + e
      const float *c = pw + 8 * s + 4;  // keys 32 s + 16 + 4 g + e
      pf[rb][s] = u32x4{pack2<kBf16>(a[0], a[1]), pack2<kBf16>(a[2], a[3]), pack2<kBf16>(c[0], c[1]),
                        pack2<kBf16>(c[2], c[3])};
    }
  }
  // O^T += V^T P^T.
#pragma unroll
  for (int db = 0; db < kDB; ++db) {
    const int dim = 16 * db + n;
    const uint16_t *vrow = vt + dim * kKT;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4 a = *reinterpret_cast<const u32x4 *>(vrow + 8 * ((4 * s + g) ^ (dim & 7)));
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) oacc[rb][db] = mfma16<kBf16>(a, pf[rb][s], oacc[rb][db]);
    }
  }
}

// Block ids: heavy query tiles (late in the prompt, more keys) first.
//   blockIdx.x = ((q_tiles - 1 - qt) * batch + b) * hkv + h) * num_splits + split
template <int kD, bool kBf16, typename BtT>
__global__ __launch_bounds__(kPThreads, 2) void paged_prefill_attention_kernel(const PrefillParams p) {
  constexpr int kKPT = kD / 64;        // keys per thread per tile (raw loads)
  constexpr int kChunks = kD / 16;     // 16-byte code chunks per row
  constexpr int kQSteps = kD / 32;     // MFMA steps over the head dims
  constexpr int kDB = kD / 16;         // 16-dim blocks of O^T
  static_assert(kKPT >= 1 && kKT * kChunks == kPThreads * kKPT, "thread map covers the tile");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  float *dec = reinterpret_cast<float *>(smem_raw);                    // [256] fp32 decode table
  float *kbias = dec + 256;                                            // [kKT] 0 or -inf per key
  uint16_t *ks = reinterpret_cast<uint16_t *>(kbias + kKT);            // [kKT][kD]
  uint16_t *vt = ks + kKT * kD;                                        // [kD][kKT]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int split = int(blockIdx.x) % p.num_splits;
  const int rest = int(blockIdx.x) / p.num_splits;
  const int h = rest % p.hkv;
  const int rb = rest / p.hkv;
  const int b = rb % p.batch;
  const int qt = p.q_tiles - 1 - rb / p.batch;
  if (request_has_images(p, b)) return;  // that request runs on the tile-image path (uniform)
  // A request's rows, clipped to the query tensor (query_start_loc is caller data).
  const int q_begin = max(p.query_start_loc[b], 0);
  const int ql = min(p.query_start_loc[b + 1], p.total_q) - q_begin;
  const int tok0 = qt * p.tokens_per_tile;
  if (tok0 >= ql) return;  // a query tile past this request's rows (uniform)
  const int kl = clamp_len(p.seq_lens[b], p.max_len);

  // This lane's query row of the S^T / O^T columns.
  const int r = wave * 16 + n;
  const int tok = tok0 + (r >> p.log2_group);
  const int qhead = h * p.group + (r & (p.group - 1));
  const bool row_ok = tok < ql;
  const int tok_last = min(tok0 + p.tokens_per_tile, ql) - 1;
  // Keys the tile can see, and this split's part of them.
  const int k_vis = p.causal ? min(kl, kl - ql + tok_last + 1) : kl;
  const int s_k0 = split * p.split_tiles * kKT;
  const int s_k1 = min(s_k0 + p.split_tiles * kKT, k_vis);
  const int ntiles = s_k1 > s_k0 ? (s_k1 - s_k0 + kKT - 1) / kKT : 0;
  // Keys of this row: [s_k0, lim).
  const int lim = !row_ok ? s_k0 : (p.causal ? min(s_k1, kl - ql + tok + 1) : s_k1);

  const size_t item = (size_t(b) * p.q_tiles + qt) * p.hkv + h;
  const size_t part = (item * p.num_splits + split) * kPRows + r;
  const size_t out_row = (size_t(q_begin + tok) * p.hq + qhead) * kD;

  // Raw rows of a tile: thread (kq, dc) loads 16-byte chunk dc of the kKPT
  // consecutive keys kq * kKPT + j (all in one cache block: block_size %
  // kKPT == 0).  Consecutive threads take consecutive key groups, so the
  // transposed V stores of one instruction fill whole V^T rows.
  constexpr int kGroups = kKT / kKPT;
  const int kq = tid % kGroups, dc = tid / kGroups;
  const BtT *bt = static_cast<const BtT *>(p.block_table) + size_t(b) * p.bt_stride;
  const int64_t rec = int64_t(p.hkv) * (kD + 4);
  // Block id of this thread's keys in the tile starting at k0 (-1: none).
  auto block_of = [&](int k0) -> int64_t {
    const int key = k0 + kq * kKPT;
    const int safe = min(key, max(p.max_len - 1, 0));  // within the table: max_len <= its capacity
    const int idx = p.log2_block_size >= 0 ? safe >> p.log2_block_size : safe / p.block_size;
    const int64_t blk = int64_t(bt[idx]);
    return key < s_k1 ? blk : int64_t(-1);
  };
  const int64_t blk_first = block_of(s_k0);  // its load needs no request length
  // Loads only: the validity of each key travels in `ok` and is applied when
  // the tile is decoded, so nothing here waits for the loads.
  u32x4 kraw[kKPT], vraw[kKPT];
  float kscl[kKPT], vscl[kKPT];
  uint32_t ok = 0;
  auto issue = [&](int k0, int64_t blk) {
    const int key0 = k0 + kq * kKPT;
    const bool blk_ok = blk >= 0 && blk < p.num_blocks;
    const int in_blk = p.log2_block_size >= 0 ? key0 & (p.block_size - 1) : key0 % p.block_size;
    const int64_t row0 = blk_ok ? (blk * p.block_size + in_blk) * rec + int64_t(h) * (kD + 4) : 0;
    ok = 0;
#pragma unroll
    for (int j = 0; j < kKPT; ++j) {
      const bool kok = blk_ok && key0 + j < s_k1;
      const int64_t off = kok ? row0 + j * rec : 0;  // absent keys read the cache's first row, then drop it
      kraw[j] = *reinterpret_cast<const u32x4_a4 *>(p.key_cache + off + 16 * dc);
      vraw[j] = *reinterpret_cast<const u32x4_a4 *>(p.value_cache + off + 16 * dc);
      kscl[j] = *reinterpret_cast<const float *>(p.key_cache + off + kD);
      vscl[j] = *reinterpret_cast<const float *>(p.value_cache + off + kD);
      ok |= uint32_t(kok) << j;
    }
  };

  // The query rows as the B operand: lane (g, n) holds dims 32 i + 8 g .. + 7 of row n.
  u32x4 qf[1][kQSteps];
  {
    const uint16_t *q = static_cast<const uint16_t *>(p.query) + out_row + 8 * g;
#pragma unroll
    for (int i = 0; i < kQSteps; ++i)
      qf[0][i] = row_ok ? *reinterpret_cast<const u32x4 *>(q + 32 * i) : u32x4{0, 0, 0, 0};
  }
  int64_t blk_next = -1;  // block id for the tile after the one in flight
  if (ntiles > 0) {
    issue(s_k0, blk_first);
    if (ntiles > 1) blk_next = block_of(s_k0 + kKT);
  }
  for (int i = tid; i < 256; i += kPThreads) dec[i] = __uint_as_float(decode_bits(uint32_t(i)));
  lds_barrier();

  f32x4_t oacc[1][kDB];
#pragma unroll
  for (int db = 0; db < kDB; ++db) oacc[0][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m[1] = {-__builtin_inff()}, l[1] = {0.f};
  const int limv[1] = {lim};

  for (int it = 0; it < ntiles; ++it) {
    const int k0 = s_k0 + it * kKT;
    decode_tile<kD, kBf16, false>(dec, kraw, vraw, kscl, vscl, ok, kq, dc, ks, vt, kbias);
    lds_barrier();
    if (it + 1 < ntiles) {  // in flight during this tile's math
      issue(k0 + kKT, blk_next);
      if (it + 2 < ntiles) blk_next = block_of(k0 + 2 * kKT);
    }

    tile_math<kD, kBf16, 1, false>(ks, vt, kbias, qf, k0, limv, p.scale_log2, n, g, m, l, oacc);
    lds_barrier();  // the tile's LDS is rewritten by the next iteration
  }

  float lt = l[0] + __shfl_xor(l[0], 16, kWave);
  lt += __shfl_xor(lt, 32, kWave);
  if (!row_ok) return;
  if (p.num_splits == 1) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t *o = static_cast<uint16_t *>(p.out) + out_row + 4 * g;
#pragma unroll
    for (int db = 0; db < kDB; ++db)
      *reinterpret_cast<u32x2 *>(o + 16 * db) =
          u32x2{pack2<kBf16>(oacc[0][db][0] * inv, oacc[0][db][1] * inv),
                pack2<kBf16>(oacc[0][db][2] * inv, oacc[0][db][3] * inv)};
  } else {
    float *po = p.part_o + part * kD + 4 * g;
    if (ntiles > 0) {
#pragma unroll
      for (int db = 0; db < kDB; ++db) *reinterpret_cast<f32x4_t *>(po + 16 * db) = oacc[0][db];
    }
    if (g == 0) {
      p.part_ml[2 * part] = ntiles > 0 ? m[0] : -__builtin_inff();
      p.part_ml[2 * part + 1] = ntiles > 0 ? lt : 0.f;
    }
  }
}

// Tile images for the prefill path (long query ranges, where every query tile
// of a (request, KV head) would decode the same pages again): workgroup
// (s, h, tile) decodes keys 64 tile .. + 63 of the request holding image slot
// s, KV head h, once into global memory in exactly the layout the attention
// step copies into LDS.  Tiles at or past the request's length are not
// written (never read).
template <int kD, bool kBf16, typename BtT>
__global__ __launch_bounds__(kPThreads) void prefill_decode_tiles_kernel(const PrefillParams p) {
  constexpr int kKPT = kD / 64;
  constexpr int kGroups = kKT / kKPT;
  constexpr uint32_t kImg = img_bytes(kD);
  static_assert(kKT * (kD / 16) == kPThreads * kKPT, "thread map covers the tile");
  __shared__ float dec[256];
  const int tid = threadIdx.x;
  const int tile = int(blockIdx.x) % p.img_tiles;
  const int bh = int(blockIdx.x) / p.img_tiles;
  const int h = bh % p.hkv, slot = bh / p.hkv;
  const int b = request_of_slot(p, slot);
  if (b < 0) return;  // an unused slot (uniform)
  const int kl = clamp_len(p.seq_lens[b], p.max_len);
  const int k0 = tile * kKT;
  if (k0 >= kl) return;  // uniform
  const int kq = tid % kGroups, dc = tid / kGroups;
  const BtT *bt = static_cast<const BtT *>(p.block_table) + size_t(b) * p.bt_stride;
  const int key0 = k0 + kq * kKPT;  // kKPT keys in one cache block: block_size % kKPT == 0
  const int safe = min(key0, p.max_len - 1);
  const int idx = p.log2_block_size >= 0 ? safe >> p.log2_block_size : safe / p.block_size;
  const int64_t blk = int64_t(bt[idx]);
  const bool blk_ok = blk >= 0 && blk < p.num_blocks;
  const int in_blk = p.log2_block_size >= 0 ? key0 & (p.block_size - 1) : key0 % p.block_size;
  const int64_t rec = int64_t(p.hkv) * (kD + 4);
  const int64_t row0 = blk_ok ? (blk * p.block_size + in_blk) * rec + int64_t(h) * (kD + 4) : 0;
  u32x4 kraw[kKPT], vraw[kKPT];
  float kscl[kKPT], vscl[kKPT];
  uint32_t ok = 0;
#pragma unroll
  for (int j = 0; j < kKPT; ++j) {
    const bool kok = blk_ok && key0 + j < kl;
    const int64_t off = kok ? row0 + j * rec : 0;  // absent keys read the cache's first row, then drop it
    kraw[j] = *reinterpret_cast<const u32x4_a4 *>(p.key_cache + off + 16 * dc);
    vraw[j] = *reinterpret_cast<const u32x4_a4 *>(p.value_cache + off + 16 * dc);
    kscl[j] = *reinterpret_cast<const float *>(p.key_cache + off + kD);
    vscl[j] = *reinterpret_cast<const float *>(p.value_cache + off + kD);
    ok |= uint32_t(kok) << j;
  }
  dec[tid] = __uint_as_float(decode_bits(uint32_t(tid)));
  lds_barrier();
  uint8_t *im = p.img + ((size_t(slot) * p.hkv + h) * p.img_tiles + tile) * kImg;
  uint16_t *ks = reinterpret_cast<uint16_t *>(im);
  decode_tile<kD, kBf16, true>(dec, kraw, vraw, kscl, vscl, ok, kq, dc, ks, ks + kKT * kD,
                         reinterpret_cast<float *>(im + 4 * kKT * kD));
}

// Prefill over tile images: a workgroup of kWaves wavefronts owns (image
// slot, KV head, query tile of 128 / G tokens, key split), 128 rows, kRB blocks of
// 16 per wavefront (every K / V^T fragment read from LDS feeds kRB MFMAs); per
// 64-key tile it copies the image into one of two LDS stages by DMA
// (global_load_lds_dwordx4, 1 KiB per instruction) while the previous tile's
// math runs, with one barrier per tile: after it, the tile has landed for
// every wavefront and every wavefront is done with the stage the next copy
// overwrites.
template <int kD, bool kBf16, int kWaves, int kRB>
__global__ __launch_bounds__(kWaves * 64) void paged_prefill_attention_img_kernel(const PrefillParams p) {
  constexpr int kDB = kD / 16;
  constexpr int kQSteps = kD / 32;
  constexpr uint32_t kImg = img_bytes(kD);
  constexpr int kCopies = int(kImg / 1024);
  static_assert(kWaves * 16 * kRB == kIRows, "rows per workgroup");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int split = int(blockIdx.x) % p.num_splits;
  const int rest = int(blockIdx.x) / p.num_splits;
  const int h = rest % p.hkv;
  const int rq = rest / p.hkv;
  const int slot = rq % p.slots;
  const int qt = p.q_tiles - 1 - rq / p.slots;
  const int b = request_of_slot(p, slot);
  if (b < 0) return;  // an unused slot (uniform)
  const int q_begin = max(p.query_start_loc[b], 0);
  const int ql = min(p.query_start_loc[b + 1], p.total_q) - q_begin;
  const int tok0 = qt * p.tokens_per_tile;
  if (tok0 >= ql) return;  // uniform
  const int kl = clamp_len(p.seq_lens[b], p.max_len);
  const int tok_last = min(tok0 + p.tokens_per_tile, ql) - 1;
  const int k_vis = p.causal ? min(kl, kl - ql + tok_last + 1) : kl;
  const int s_k0 = split * p.split_tiles * kKT;
  const int s_k1 = min(s_k0 + p.split_tiles * kKT, k_vis);
  const int ntiles = s_k1 > s_k0 ? (s_k1 - s_k0 + kKT - 1) / kKT : 0;
  const size_t item = (size_t(slot) * p.q_tiles + qt) * p.hkv + h;
  // Row block rb of this wavefront: rows 16 (kRB wave + rb) + n.
  int r[kRB], tok[kRB], lim[kRB];
  bool row_ok[kRB];
  size_t out_row[kRB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    r[rb] = (wave * kRB + rb) * 16 + n;
    tok[rb] = tok0 + (r[rb] >> p.log2_group);
    row_ok[rb] = tok[rb] < ql;
    lim[rb] = !row_ok[rb] ? s_k0 : (p.causal ? min(s_k1, kl - ql + tok[rb] + 1) : s_k1);
    const int qhead = h * p.group + (r[rb] & (p.group - 1));
    out_row[rb] = (size_t(q_begin + tok[rb]) * p.hq + qhead) * kD;
  }

  // Tile t of this (request, KV head) lands in stage s: copy instruction j
  // (wavefront j % kWaves) moves bytes 1024 j .. + 1023, lane i 16 of them.
  const uint8_t *img = p.img + (size_t(slot) * p.hkv + h) * p.img_tiles * kImg + 16 * lane;
  const uint32_t lds0 = lds_address(smem_raw);
  const int t0 = s_k0 / kKT;
  auto copy = [&](int t, int stage) {
    const uint8_t *src = img + size_t(t) * kImg;
    for (int j = wave; j < kCopies; j += kWaves) dma16(src + 1024 * j, lds0 + uint32_t(stage) * kImg + 1024u * j);
  };
  u32x4 qf[kRB][kQSteps];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const uint16_t *q = static_cast<const uint16_t *>(p.query) + out_row[rb] + 8 * g;
#pragma unroll
    for (int i = 0; i < kQSteps; ++i)
      qf[rb][i] = row_ok[rb] ? *reinterpret_cast<const u32x4 *>(q + 32 * i) : u32x4{0, 0, 0, 0};
  }
  if (ntiles > 0) copy(t0, 0);
  f32x4_t oacc[kRB][kDB];
  float m[kRB], l[kRB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    m[rb] = -__builtin_inff();
    l[rb] = 0.f;
#pragma unroll
    for (int db = 0; db < kDB; ++db) oacc[rb][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // The smallest key limit of the wavefront's rows: tiles wholly below it
  // need no mask.
  int lim_lo = lim[0];
#pragma unroll
  for (int rb = 1; rb < kRB; ++rb) lim_lo = min(lim_lo, lim[rb]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) lim_lo = min(lim_lo, __shfl_xor(lim_lo, off, kWave));
  lim_lo = __builtin_amdgcn_readfirstlane(lim_lo);
  for (int it = 0; it < ntiles; ++it) {
    wait_vmcnt<0>();  // this wavefront's copies of tile it (the only ones in flight)
    lds_barrier();
    if (it + 1 < ntiles) copy(t0 + it + 1, (it + 1) & 1);
    const uint8_t *st = smem_raw + (it & 1) * kImg;
    const uint16_t *ks = reinterpret_cast<const uint16_t *>(st);
    const int k0 = s_k0 + it * kKT;
    tile_math<kD, kBf16, kRB, true>(ks, ks + kKT * kD, reinterpret_cast<const float *>(st + 4 * kKT * kD), qf, k0,
                              lim, p.scale_log2, n, g, m, l, oacc, k0 + kKT <= lim_lo);
  }

#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    float lt = l[rb] + __shfl_xor(l[rb], 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    if (!row_ok[rb]) continue;
    if (p.num_splits == 1) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      uint16_t *o = static_cast<uint16_t *>(p.out) + out_row[rb] + 4 * g;
#pragma unroll
      for (int db = 0; db < kDB; ++db)
        *reinterpret_cast<u32x2 *>(o + 16 * db) = u32x2{pack2<kBf16>(oacc[rb][db][0] * inv, oacc[rb][db][1] * inv),
                                                        pack2<kBf16>(oacc[rb][db][2] * inv, oacc[rb][db][3] * inv)};
    } else {
      const size_t part = (item * p.num_splits + split) * kIRows + r[rb];
      float *po = p.part_o + part * kD + 4 * g;
      if (ntiles > 0) {
#pragma unroll
        for (int db = 0; db < kDB; ++db) *reinterpret_cast<f32x4_t *>(po + 16 * db) = oacc[rb][db];
      }
      if (g == 0) {
        p.part_ml[2 * part] = ntiles > 0 ? m[rb] : -__builtin_inff();
        p.part_ml[2 * part + 1] = ntiles > 0 ? lt : 0.f;
      }
    }
  }
}

// Merges the key splits of each (query tile, KV head) row:
//   M = max_s m_s, w_s = 2^(m_s - M), out = sum_s w_s O_s / sum_s w_s l_s,
// splits added in order.  One wavefront per row, four rows per workgroup:
// lane s reads split s's (m, l); then each lane adds its four output dims of
// every split, eight splits' loads issued before their adds.  Splits with
// weight 0 (no key) are skipped, so their unwritten partial outputs are
// never read.  (One workgroup per row with the splits spread over four
// wavefronts measured 11.7 us for 8192 rows of 4 splits.)
constexpr int kMaxCombineSplits = 64;

// kSlots: the items are (image slot, query tile, KV head) of the tile-image
// path; otherwise (request, query tile, KV head) of the in-kernel path.
template <bool kBf16, int kRows, bool kSlots>
__global__ __launch_bounds__(kPThreads) void prefill_combine_kernel(const PrefillParams p) {
  const int item = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int r = int(blockIdx.y) * (kPThreads / kWave) + (threadIdx.x >> 6);
  const int h = item % p.hkv;
  const int qt = (item / p.hkv) % p.q_tiles;
  const int rq = item / (p.hkv * p.q_tiles);
  const int b = kSlots ? request_of_slot(p, rq) : rq;
  if (b < 0 || (!kSlots && request_has_images(p, b))) return;  // uniform
  const int q_begin = max(p.query_start_loc[b], 0);
  const int ql = min(p.query_start_loc[b + 1], p.total_q) - q_begin;
  const int tok = qt * p.tokens_per_tile + (r >> p.log2_group);
  if (r >= kRows || tok >= ql) return;  // wavefront-uniform: a row past the request
  const size_t base = size_t(item) * p.num_splits * kRows + r;  // part index of split 0
  const bool have = lane < p.num_splits;
  const size_t pi = base + size_t(have ? lane : 0) * kRows;
  const float ms = have ? p.part_ml[2 * pi] : -__builtin_inff();
  const float ls = have ? p.part_ml[2 * pi + 1] : 0.f;
  const float mx = wave_max(ms);
  const float w = ms == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
  const float total = wave_sum(w * ls);
  const bool dims_ok = 4 * lane < p.dv;
  f32x4_t acc{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < p.num_splits; s0 += 8) {
    float ws[8];
    f32x4_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int s = s0 + j;
      ws[j] = __shfl(w, s < p.num_splits ? s : 0, kWave);  // every lane active here
      if (s >= p.num_splits) ws[j] = 0.f;
      v[j] = dims_ok && ws[j] != 0.f
                 ? *reinterpret_cast<const f32x4_t *>(p.part_o + (base + size_t(s) * kRows) * p.dv + 4 * lane)
                 : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += ws[j] * v[j];
  }
  if (!dims_ok) return;
  const float inv = total > 0.f ? 1.f / total : 0.f;
  const int qhead = h * p.group + (r & (p.group - 1));
  uint16_t *o = static_cast<uint16_t *>(p.out) + (size_t(q_begin + tok) * p.hq + qhead) * p.dv + 4 * lane;
  *reinterpret_cast<u32x2 *>(o) = u32x2{pack2<kBf16>(acc[0] * inv, acc[1] * inv), pack2<kBf16>(acc[2] * inv, acc[3] * inv)};
}

// Any head sizes, group or block size: one wavefront per (query row, query
// head), keys one at a time with the online softmax; K and V rounded to the
// query dtype like the MFMA kernel.
template <bool kBf16, typename BtT>
__global__ __launch_bounds__(kWave) void paged_prefill_attention_simple(const PrefillParams p, int total_q) {
  const int row = int(blockIdx.x) / p.hq, head = int(blockIdx.x) % p.hq;
  if (row >= total_q) return;
  // The request of this query row: the last b with query_start_loc[b] <= row.
  int lo = 0, hi = p.batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (p.query_start_loc[mid] <= row) lo = mid;
    else hi = mid - 1;
  }
  const int b = lo;
  const int q_begin = p.query_start_loc[b];
  const int ql = p.query_start_loc[b + 1] - q_begin;
  if (row < q_begin || row - q_begin >= ql) return;  // rows outside every request
  const int kl = clamp_len(p.seq_lens[b], p.max_len);
  const int lim = p.causal ? min(kl, kl - ql + (row - q_begin) + 1) : kl;
  const int h = head / p.group;
  const int lane = threadIdx.x;
  const uint16_t *q = static_cast<const uint16_t *>(p.query) + (size_t(row) * p.hq + head) * p.d;
  const BtT *bt = static_cast<const BtT *>(p.block_table) + size_t(b) * p.bt_stride;
  const int64_t krow = p.d + 4, vrow = p.dv + 4;
  constexpr int kMaxPerLane = 8;  // head sizes up to 512
  float qv[kMaxPerLane], acc[kMaxPerLane];
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int dim = lane + kWave * i;
    qv[i] = dim < p.d ? half_bits_to_float<kBf16>(q[dim]) : 0.f;
    acc[i] = 0.f;
  }
  float m = -__builtin_inff(), l = 0.f;
  for (int t = 0; t < lim; ++t) {
    const int64_t blk = int64_t(bt[t / p.block_size]);
    if (blk < 0 || blk >= p.num_blocks) continue;
    const int64_t slot = blk * p.block_size + t % p.block_size;
    const uint8_t *kr = p.key_cache + (slot * p.hkv + h) * krow;
    const uint8_t *vr = p.value_cache + (slot * p.hkv + h) * vrow;
    const float ksc = *reinterpret_cast<const float *>(kr + p.d);
    const float vsc = *reinterpret_cast<const float *>(vr + p.dv);
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      const int dim = lane + kWave * i;
      if (dim < p.d)
        dot = fmaf(qv[i], half_bits_to_float<kBf16>(float_to_half_bits<kBf16>(
                              __uint_as_float(kDeviceTables.decode_f32[kr[dim]]) * ksc)), dot);
    }
    dot = wave_sum(dot);
    const float x = dot * p.scale_log2;
    const float m_new = fmaxf(m, x);
    const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    const float pw = __builtin_amdgcn_exp2f(x - m_use);
    l = l * alpha + pw;
    m = m_new;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      const int dim = lane + kWave * i;
      acc[i] *= alpha;
      if (dim < p.dv)
        acc[i] = fmaf(pw, half_bits_to_float<kBf16>(float_to_half_bits<kBf16>(
                              __uint_as_float(kDeviceTables.decode_f32[vr[dim]]) * vsc)), acc[i]);
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t *o = static_cast<uint16_t *>(p.out) + (size_t(row) * p.hq + head) * p.dv;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int dim = lane + kWave * i;
    if (dim < p.dv) o[dim] = float_to_half_bits<kBf16>(acc[i] * inv);
  }
}

// ------------------------------------------------------------- host side

int log2_exact(int64_t v) {
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return (int64_t(1) << l) == v ? l : -1;
}

bool prefill_mfma_shape(int64_t d, int64_t dv, int64_t group, int64_t block_size) {
  return (d == 64 || d == 128 || d == 256) && dv == d && group >= 1 && group <= 16 && log2_exact(group) >= 0 &&
         block_size % 4 == 0;
}

struct PrefillPlan {
  int tokens_per_tile, q_tiles, num_splits, split_tiles;
  int rows;  // (token, head) rows per workgroup
};

// One path's plan over `requests` request slots of the grid whose longest
// query has q_cover tokens: query tiles of rows / G tokens; key splits while
// the (request, query tile, KV head) items leave fewer than ~512 (in-kernel
// path) or ~256 (images, one eight-wave workgroup per CU) workgroups, each
// split at least two 64-key tiles.
PrefillPlan plan_path(int64_t requests, int64_t hkv, int64_t group, int64_t q_cover, int64_t max_len, bool img) {
  PrefillPlan pl{};
  const int64_t kv_tiles = std::max<int64_t>((max_len + kKT - 1) / kKT, 1);
  pl.rows = img ? kIRows : kPRows;
  pl.tokens_per_tile = int(pl.rows / group);
  pl.q_tiles = int((std::max<int64_t>(q_cover, 1) + pl.tokens_per_tile - 1) / pl.tokens_per_tile);
  const int64_t items = std::max<int64_t>(requests, 1) * pl.q_tiles * hkv;
  const int64_t target = img ? kITargetBlocks : kTargetBlocks;
  int64_t splits = (target + items - 1) / items;
  if (splits > kv_tiles) splits = kv_tiles;
  if (splits < 1) splits = 1;
  int64_t per = (kv_tiles + splits - 1) / splits;
  if (per < kMinSplitTiles) per = std::min<int64_t>(kMinSplitTiles, kv_tiles);
  if ((kv_tiles + per - 1) / per > kMaxCombineSplits) per = (kv_tiles + kMaxCombineSplits - 1) / kMaxCombineSplits;
  pl.split_tiles = int(per);
  pl.num_splits = int((kv_tiles + per - 1) / per);
  return pl;
}

// Image bytes the tile-image path may hold per call (512 MiB, or
// HIF8_PREFILL_IMAGE_CAP_MB, read at every call); long requests beyond the
// slots this buys take the in-kernel path.
int64_t image_cap_bytes() {
  const char *v = getenv("HIF8_PREFILL_IMAGE_CAP_MB");
  const int64_t mb = v && *v ? atoll(v) : 512;
  return (mb > 0 ? mb : 0) << 20;
}

// Both paths of one call.  A request runs on the tile-image path when its
// query covers more than two 64-row tiles (every page would otherwise be
// decoded once per query tile; measured on MI355X, 512 rows over 4096 keys:
// B=4 461 -> 214 us) and it gets an image slot; up to two tiles the
// in-kernel decode is as fast or faster (17 rows x 4 heads over 4096 keys:
// B=1 29.6 vs 29.1 us, B=4 47.1 vs 55.6 us with images).  Slots: at most one
// per request that can be long (total_q / (long_rows / G + 1) of them), within
// image_cap_bytes().  When every long request has a slot, the in-kernel path
// covers only the short ones (two query tiles).
struct PrefillPlans {
  PrefillPlan in, img;
  int slots, long_rows, img_tiles;
};

PrefillPlans plan_prefill(int64_t batch, int64_t hkv, int64_t group, int64_t total_q, int64_t max_query_len,
                          int64_t max_len, int d) {
  static const int img_env = [] {
    const char *v = getenv("HIF8_PREFILL_IMAGES");  // tuning: 0 never, 1 for every multi-tile query
    return v && *v ? atoi(v) : -1;
  }();
  PrefillPlans pp{};
  const int64_t kv_tiles = std::max<int64_t>((max_len + kKT - 1) / kKT, 1);
  pp.long_rows = img_env == 1 ? kPRows : 2 * kPRows;
  int64_t long_max = 0;
  if (img_env != 0 && std::max<int64_t>(max_query_len, 1) * group > pp.long_rows) {
    long_max = std::min<int64_t>(batch, total_q / (pp.long_rows / group + 1));
    const int64_t per_slot = hkv * kv_tiles * int64_t(img_bytes(d));
    pp.slots = int(std::min<int64_t>(long_max, std::max<int64_t>(1, image_cap_bytes() / per_slot)));
  }
  pp.img_tiles = pp.slots > 0 ? int(kv_tiles) : 0;
  if (pp.slots > 0) pp.img = plan_path(pp.slots, hkv, group, max_query_len, max_len, true);
  const int64_t in_cover =
      pp.slots > 0 && pp.slots >= long_max ? std::min<int64_t>(max_query_len, pp.long_rows / group) : max_query_len;
  pp.in = plan_path(batch, hkv, group, in_cover, max_len, false);
  return pp;
}

// Workspace bytes: images, the image path's split partials, the in-kernel
// path's split partials (each partial region: outputs, then (max, sum)).
struct PrefillWorkspace {
  size_t images, img_parts, in_parts;
};

PrefillWorkspace prefill_workspace(const PrefillPlans &pp, int64_t batch, int64_t hkv, int d, int dv) {
  PrefillWorkspace w{};
  w.images = size_t(pp.slots) * hkv * pp.img_tiles * img_bytes(d);
  if (pp.slots > 0 && pp.img.num_splits > 1)
    w.img_parts = size_t(pp.slots) * pp.img.q_tiles * hkv * pp.img.num_splits * pp.img.rows * size_t(dv + 2) * 4;
  if (pp.in.num_splits > 1)
    w.in_parts = size_t(batch) * pp.in.q_tiles * hkv * pp.in.num_splits * pp.in.rows * size_t(dv + 2) * 4;
  return w;
}

size_t prefill_smem(int d) { return size_t(256 + kKT) * 4 + size_t(2) * kKT * d * 2; }

template <int kD, bool kBf16, typename BtT>
int launch_prefill_mfma(const PrefillParams &p, hipStream_t stream) {
  const void *fn = reinterpret_cast<const void *>(&paged_prefill_attention_kernel<kD, kBf16, BtT>);
  const size_t smem = prefill_smem(kD);
  if (const int st = reserve_dynamic_lds(fn, smem, "hif8_paged_prefill_attention")) return st;
  const unsigned blocks = unsigned(int64_t(p.q_tiles) * p.batch * p.hkv * p.num_splits);
  paged_prefill_attention_kernel<kD, kBf16, BtT><<<blocks, kPThreads, smem, stream>>>(p);
  if (p.num_splits > 1)
    prefill_combine_kernel<kBf16, kPRows, false>
        <<<dim3(unsigned(int64_t(p.batch) * p.q_tiles * p.hkv), kPRows / (kPThreads / kWave)), kPThreads, 0, stream>>>(p);
  return HIF8_OK;
}

template <int kD, bool kBf16, typename BtT>
int launch_prefill_img(const PrefillParams &p, hipStream_t stream) {
  prefill_decode_tiles_kernel<kD, kBf16, BtT>
      <<<unsigned(int64_t(p.slots) * p.hkv * p.img_tiles), kPThreads, 0, stream>>>(p);
  // Eight wavefronts of one 16-row block each.  Four wavefronts of two
  // blocks (half the LDS fragment reads per row, one wavefront per SIMD)
  // measured slower on MI355X: 512 rows over 4096 keys, B=4 310 vs 214 us.
  const size_t smem = 2 * size_t(img_bytes(kD));
  const unsigned blocks = unsigned(int64_t(p.q_tiles) * p.slots * p.hkv * p.num_splits);
  const auto kern = &paged_prefill_attention_img_kernel<kD, kBf16, kIWaves, 1>;
  if (const int st = reserve_dynamic_lds(reinterpret_cast<const void *>(kern), smem, "hif8_paged_prefill_attention"))
    return st;
  kern<<<blocks, kIThreads, smem, stream>>>(p);
  if (p.num_splits > 1)
    prefill_combine_kernel<kBf16, kIRows, true>
        <<<dim3(unsigned(int64_t(p.slots) * p.q_tiles * p.hkv), kIRows / (kPThreads / kWave)), kPThreads, 0, stream>>>(p);
  return HIF8_OK;
}

// p_in: the in-kernel path (every request without an image slot); p_img
// (p_img.slots > 0): the tile-image path.  The two write disjoint rows.
template <bool kBf16, typename BtT>
int launch_prefill(const PrefillParams &p_in, const PrefillParams &p_img, bool mfma, int64_t total_q,
                   hipStream_t stream) {
  if (!mfma) {
    paged_prefill_attention_simple<kBf16, BtT><<<unsigned(total_q * p_in.hq), kWave, 0, stream>>>(p_in, int(total_q));
    return HIF8_OK;
  }
  if (p_img.slots > 0) {
    int st;
    switch (p_img.d) {
      case 64: st = launch_prefill_img<64, kBf16, BtT>(p_img, stream); break;
      case 128: st = launch_prefill_img<128, kBf16, BtT>(p_img, stream); break;
      default: st = launch_prefill_img<256, kBf16, BtT>(p_img, stream); break;
    }
    if (st) return st;
  }
  switch (p_in.d) {
    case 64: return launch_prefill_mfma<64, kBf16, BtT>(p_in, stream);
    case 128: return launch_prefill_mfma<128, kBf16, BtT>(p_in, stream);
    default: return launch_prefill_mfma<256, kBf16, BtT>(p_in, stream);
  }
}

}  // namespace
}  // namespace hif8

using namespace hif8;

extern "C" size_t hif8_paged_prefill_attention_workspace_size(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                                              int64_t head_size, int64_t head_size_v,
                                                              int64_t total_query_tokens, int64_t max_query_len,
                                                              int64_t max_seq_len) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 || head_size_v <= 0 ||
      total_query_tokens <= 0 || max_query_len <= 0 || max_seq_len <= 0 || num_heads % num_kv_heads)
    return 0;
  const int64_t group = num_heads / num_kv_heads;
  if (!prefill_mfma_shape(head_size, head_size_v, group, 4)) return 0;  // the simple kernel needs none
  const PrefillPlans pp =
      plan_prefill(batch, num_kv_heads, group, total_query_tokens, max_query_len, max_seq_len, int(head_size));
  const PrefillWorkspace w = prefill_workspace(pp, batch, num_kv_heads, int(head_size), int(head_size_v));
  return w.images + w.img_parts + w.in_parts;
}

extern "C" int hif8_paged_prefill_attention(const void *query, int q_dtype, const uint8_t *key_cache,
                                            const uint8_t *value_cache, int64_t num_blocks, int64_t block_size,
                                            int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
                                            const void *block_table, int block_table_dtype,
                                            int64_t max_blocks_per_seq, const int32_t *query_start_loc,
                                            const int32_t *seq_lens, int64_t batch, int64_t num_heads,
                                            int64_t total_query_tokens, int64_t max_query_len, int64_t max_seq_len,
                                            float scale, int causal, void *out, void *workspace,
                                            size_t workspace_bytes, hif8_stream_t stream) {
  clear_error();
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 || head_size_v <= 0 ||
      num_blocks <= 0 || block_size <= 0 || max_blocks_per_seq <= 0 || max_seq_len < 0 || max_query_len < 0 ||
      total_query_tokens < 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: dimensions must be positive");
  if (num_heads % num_kv_heads)
    return fail(HIF8_ERR_INVALID_ARGUMENT,
                "hif8_paged_prefill_attention: num_heads must be divisible by num_kv_heads");
  if (head_size % 4 || head_size_v % 4)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: head sizes must be divisible by four");
  if (head_size > 512 || head_size_v > 512)
    return fail(HIF8_ERR_UNSUPPORTED, "hif8_paged_prefill_attention: head sizes above 512 are not supported");
  if (!is_io_dtype(q_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: query must be float16 or bfloat16");
  if (block_table_dtype != HIF8_INDEX_INT32 && block_table_dtype != HIF8_INDEX_INT64)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: block_table must be int32 or int64");
  if (max_seq_len > max_blocks_per_seq * block_size)
    return fail(HIF8_ERR_INVALID_ARGUMENT,
                "hif8_paged_prefill_attention: max_seq_len exceeds the block table capacity");
  if (max_seq_len > 0x7FFFFFFFll || batch > 0x7FFFFFFFll || num_heads > 0xFFFF ||
      total_query_tokens * num_heads > 0x7FFFFFFFll || max_query_len > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: dimensions too large");
  if (batch == 0 || total_query_tokens == 0) return HIF8_OK;
  if (max_query_len == 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: max_query_len must cover the query rows");
  if (!query || !key_cache || !value_cache || !block_table || !query_start_loc || !seq_lens || !out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: null pointer argument");
  if (!aligned(key_cache, 4) || !aligned(value_cache, 4))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: caches must be 4-byte aligned");
  if (!aligned(query, 2) || !aligned(out, 2))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: query/out must be 2-byte aligned");

  PrefillParams p{};
  p.query = query;
  p.key_cache = key_cache;
  p.value_cache = value_cache;
  p.block_table = block_table;
  p.query_start_loc = query_start_loc;
  p.seq_lens = seq_lens;
  p.out = out;
  p.bt_stride = max_blocks_per_seq;
  p.num_blocks = num_blocks;
  p.block_size = int(block_size);
  p.log2_block_size = log2_exact(block_size);
  p.hkv = int(num_kv_heads);
  p.hq = int(num_heads);
  p.group = int(num_heads / num_kv_heads);
  p.d = int(head_size);
  p.dv = int(head_size_v);
  p.batch = int(batch);
  p.max_len = int(max_seq_len);
  p.causal = causal ? 1 : 0;
  p.total_q = int(total_query_tokens);
  p.scale_log2 = scale * 1.4426950408889634f;
  const bool mfma = prefill_mfma_shape(head_size, head_size_v, p.group, block_size) && aligned(query, 16) &&
                    aligned(out, 16);
  PrefillParams pi = p;  // the tile-image path
  p.log2_group = log2_exact(p.group);
  if (mfma) {
    const PrefillPlans pp =
        plan_prefill(batch, num_kv_heads, p.group, total_query_tokens, max_query_len, max_seq_len, int(head_size));
    auto apply = [](PrefillParams &q, const PrefillPlan &pl) {
      q.tokens_per_tile = pl.tokens_per_tile;
      q.q_tiles = pl.q_tiles;
      q.num_splits = pl.num_splits;
      q.split_tiles = pl.split_tiles;
    };
    p.slots = pp.slots;
    p.long_rows = pp.long_rows;
    apply(p, pp.in);
    pi = p;
    if (pp.slots > 0) apply(pi, pp.img);
    pi.img_tiles = pp.img_tiles;
    if (int64_t(p.q_tiles) * batch * num_kv_heads * p.num_splits > 0x7FFFFFFFll ||
        int64_t(pi.q_tiles) * pp.slots * num_kv_heads * pi.num_splits > 0x7FFFFFFFll ||
        int64_t(pp.slots) * num_kv_heads * pp.img_tiles > 0x7FFFFFFFll)
      return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: too many query tiles");
    const PrefillWorkspace w = prefill_workspace(pp, batch, num_kv_heads, int(head_size), int(head_size_v));
    const size_t need = w.images + w.img_parts + w.in_parts;
    if (need > 0) {
      if (!workspace || workspace_bytes < need)
        return fail(HIF8_ERR_INVALID_ARGUMENT,
                    "hif8_paged_prefill_attention: workspace of %zu bytes required (got %zu)", need,
                    workspace_bytes);
      if (!aligned(workspace, 16))
        return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_prefill_attention: workspace must be 16-byte aligned");
      uint8_t *ws = static_cast<uint8_t *>(workspace);
      if (pp.slots > 0) pi.img = ws;
      if (w.img_parts) {
        pi.part_o = reinterpret_cast<float *>(ws + w.images);
        pi.part_ml = pi.part_o + size_t(pp.slots) * pi.q_tiles * num_kv_heads * pi.num_splits * kIRows * head_size_v;
      }
      if (w.in_parts) {
        p.part_o = reinterpret_cast<float *>(ws + w.images + w.img_parts);
        p.part_ml = p.part_o + size_t(batch) * p.q_tiles * num_kv_heads * p.num_splits * kPRows * head_size_v;
      }
    }
  } else {
    p.log2_group = 0;
    p.tokens_per_tile = 1;
    p.q_tiles = 1;
    p.num_splits = 1;
    p.split_tiles = 1;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf16 = q_dtype == HIF8_DTYPE_BF16, i64 = block_table_dtype == HIF8_INDEX_INT64;
  int st;
  if (bf16 && i64) st = launch_prefill<true, int64_t>(p, pi, mfma, total_query_tokens, s);
  else if (bf16) st = launch_prefill<true, int32_t>(p, pi, mfma, total_query_tokens, s);
  else if (i64) st = launch_prefill<false, int64_t>(p, pi, mfma, total_query_tokens, s);
  else st = launch_prefill<false, int32_t>(p, pi, mfma, total_query_tokens, s);
  if (st) return st;
  return check_launch("hif8_paged_prefill_attention");
}
