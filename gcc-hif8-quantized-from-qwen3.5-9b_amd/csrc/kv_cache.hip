// HiF8 paged KV cache for gfx950: the fused static cache write and the
// split-context decode attention that decodes cache pages inside the kernel.
//
// Cache layout (kv_cache.py:26-88): K and V are separate uint8 tensors
// [num_blocks, block_size, Hkv, D + 4]; a row is D HiF8 codes followed by its
// FP32 scale, little-endian (kv_cache.py:151-170).  The Hkv rows of one token
// are contiguous (a "record" of Hkv * (D + 4) bytes), and token t of a request
// lives in flat slot block_table[t / block_size] * block_size + t % block_size.
//
// Write (kv_runtime.py:1168-1199, 1222-1339): row (t, h) holds
// static_encode(x[t, h, :] / scale[h]) and the sidecar scale[h]; slot < 0 is a
// padding token and is skipped.  One thread encodes 16 codes with the same
// encoder as hif8_static_quant, so the bytes equal quant -> pack -> scatter.
//
// Decode attention (kv_runtime.py:1470-1563 semantics, oracle kv_cache.py:314-372):
// one query token per request, GQA group G = Hq / Hkv.  A workgroup owns one
// request's token range (a "split") and four KV heads, one wavefront each; a
// wavefront walks its range in 32-token tiles:
//   * K rows go from HBM straight into VGPRs in the MFMA A-operand layout
//     (token = lane % 16, 64 contiguous bytes per lane), are decoded through a
//     256-entry table in LDS, and S^T = K Q^T runs on v_mfma_f32_16x16x32
//     (B = the G query heads of the KV head, padded to 16 columns);
//   * V rows are staged raw in LDS and read transposed (8 tokens x 4 dims per
//     lane), decoded, and O^T += V^T P' runs on the same MFMA with the
//     softmax weights P' rounded to bf16;
//   * rows with the head's scale (static caches) decode through per-head tables
//     of bf16/fp16(dec(c) * scale), i.e. rounded like the reference's decoded
//     K/V; rows with other scales decode exactly and the K row scale and
//     V row scale multiply the logits and softmax weights in FP32 instead;
//   * the online softmax keeps (max, sum) per query head in FP32;
//   * the next tile's loads are in flight while the current tile computes.
// HiF8 values are exact in bf16 and fp16, so decode adds no rounding.  With
// more than one split per request, partial (O, max, sum) go to the caller's
// workspace and a second kernel merges them.
#include <stdlib.h>

#include "quant_device.h"

namespace hif8 {
namespace {

constexpr int kThreads = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Cache rows are (D + 4) bytes long, so row data is only 4-byte aligned.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

int grid_for(uint64_t work_items, int per_cu) {
  uint64_t blocks = (work_items + kThreads - 1) / kThreads;
  const uint64_t cap = uint64_t(256) * per_cu;  // 256 CUs on MI355X
  if (blocks > cap) blocks = cap;
  return int(blocks < 1 ? 1 : blocks);
}

// ------------------------------------------------------------------ write

// One thread = 16 codes of one row.  Items are token-major with the token's
// K rows before its V rows, so a wavefront writes whole contiguous rows.
template <bool kBf16, typename SlotT>
__global__ __launch_bounds__(kThreads) void kv_write_vec16(
    const uint16_t *__restrict__ key, const uint16_t *__restrict__ value,
    const float *__restrict__ key_scale, const float *__restrict__ value_scale,
    const SlotT *__restrict__ slots, uint8_t *__restrict__ key_cache,
    uint8_t *__restrict__ value_cache, uint32_t tokens, uint32_t hkv, uint32_t d, uint32_t dv,
    uint64_t capacity, int32_t *__restrict__ invalid) {
  __shared__ __attribute__((aligned(16))) uint8_t lut[8192];
  stage_static_encode_table(lut, threadIdx.x, kThreads);
  __syncthreads();
  const uint32_t k_items = hkv * (d / 16);
  const uint32_t per_token = k_items + hkv * (dv / 16);
  const uint64_t total = uint64_t(tokens) * per_token;
  const uint64_t stride = uint64_t(gridDim.x) * kThreads;
  for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < total; i += stride) {
    const uint32_t t = uint32_t(i / per_token);
    uint32_t r = uint32_t(i - uint64_t(t) * per_token);
    const bool is_v = r >= k_items;
    if (is_v) r -= k_items;
    const uint32_t width = is_v ? dv : d;
    const uint32_t h = r / (width / 16), col = r - h * (width / 16);
    const int64_t slot = int64_t(slots[t]);
    if (slot < 0) continue;  // padding token
    if (uint64_t(slot) >= capacity) {
      if (invalid && r == 0 && !is_v) atomicAdd(invalid, 1);
      continue;
    }
    float xf[16];
    load16<kBf16>((is_v ? value : key) + (size_t(t) * hkv + h) * width + 16 * col, xf);
    const float s = (is_v ? value_scale : key_scale)[h];
    uint32_t w[4];
    static_encode16(xf, s, lut, w);
    uint8_t *row = (is_v ? value_cache : key_cache) + (uint64_t(slot) * hkv + h) * (width + 4);
    *reinterpret_cast<u32x4_a4 *>(row + 16 * col) = u32x4{w[0], w[1], w[2], w[3]};
    if (col == 0) *reinterpret_cast<float *>(row + width) = s;
  }
}

// Any head size divisible by 4 and any alignment: one thread per code,
// IEEE division and the arithmetic static encoder.
template <bool kBf16, typename SlotT>
__global__ __launch_bounds__(kThreads) void kv_write_scalar(
    const uint16_t *__restrict__ key, const uint16_t *__restrict__ value,
    const float *__restrict__ key_scale, const float *__restrict__ value_scale,
    const SlotT *__restrict__ slots, uint8_t *__restrict__ key_cache,
    uint8_t *__restrict__ value_cache, uint32_t tokens, uint32_t hkv, uint32_t d, uint32_t dv,
    uint64_t capacity, int32_t *__restrict__ invalid) {
  const uint32_t k_items = hkv * d;
  const uint32_t per_token = k_items + hkv * dv;
  const uint64_t total = uint64_t(tokens) * per_token;
  const uint64_t stride = uint64_t(gridDim.x) * kThreads;
  for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < total; i += stride) {
    const uint32_t t = uint32_t(i / per_token);
    uint32_t r = uint32_t(i - uint64_t(t) * per_token);
    const bool is_v = r >= k_items;
    if (is_v) r -= k_items;
    const uint32_t width = is_v ? dv : d;
    const uint32_t h = r / width, col = r - h * width;
    const int64_t slot = int64_t(slots[t]);
    if (slot < 0) continue;
    if (uint64_t(slot) >= capacity) {
      if (invalid && r == 0 && !is_v) atomicAdd(invalid, 1);
      continue;
    }
    const float s = (is_v ? value_scale : key_scale)[h];
    const uint16_t x = (is_v ? value : key)[(size_t(t) * hkv + h) * width + col];
    const float q = half_bits_to_float<kBf16>(x) / s;
    uint8_t *row = (is_v ? value_cache : key_cache) + (uint64_t(slot) * hkv + h) * (width + 4);
    row[col] = uint8_t(static_encode_bits(__float_as_uint(q)));
    if (col == 0) *reinterpret_cast<float *>(row + width) = s;
  }
}

// -------------------------------------------------------------- attention

constexpr int kTile = 32;        // tokens per tile: two 16-row MFMA blocks
constexpr int kWaves = 4;        // KV heads per workgroup, one wavefront each
constexpr int kMaxSplits = 4096; // combine kernel's LDS weight array

struct AttnParams {
  const void *query;          // [B, Hq, D]
  const uint8_t *key_cache;   // [num_blocks, block_size, Hkv, D + 4]
  const uint8_t *value_cache; // [num_blocks, block_size, Hkv, Dv + 4]
  const void *block_table;    // [B, bt_stride] int32 or int64
  const int32_t *seq_lens;    // [B]
  void *out;                  // [B, Hq, Dv]
  float *part_o;              // [B, num_splits, Hq, Dv]
  float *part_ml;             // [B, num_splits, Hq, 2]
  int64_t bt_stride;
  int64_t num_blocks;
  int block_size, hkv, hq, group, d, dv;
  int max_len, split_tokens, num_splits;
  float scale_log2;           // softmax scale * log2(e)
};

__device__ __forceinline__ int clamp_len(int len, int max_len) {
  return len < 0 ? 0 : (len > max_len ? max_len : len);
}

// Two table entries packed as one 16-bit pair (one v_perm_b32).
__device__ __forceinline__ uint32_t lut_pair(const uint16_t *lut, uint32_t lo, uint32_t hi) {
  u16x2 v;
  v.x = lut[lo];
  v.y = lut[hi];
  return __builtin_bit_cast(uint32_t, v);
}

// Eight codes (two little-endian words) -> an MFMA operand of eight 16-bit values.
__device__ __forceinline__ u32x4 decode8(const uint16_t *lut, uint32_t w0, uint32_t w1) {
  return u32x4{lut_pair(lut, w0 & 0xFFu, (w0 >> 8) & 0xFFu), lut_pair(lut, (w0 >> 16) & 0xFFu, w0 >> 24),
               lut_pair(lut, w1 & 0xFFu, (w1 >> 8) & 0xFFu), lut_pair(lut, (w1 >> 16) & 0xFFu, w1 >> 24)};
}

// Byte q of each of eight words -> operand (element j from word j).
__device__ __forceinline__ u32x4 decode_column(const uint16_t *lut, const uint32_t (&w)[8], int q) {
  const int sh = 8 * q;
  return u32x4{lut_pair(lut, (w[0] >> sh) & 0xFFu, (w[1] >> sh) & 0xFFu),
               lut_pair(lut, (w[2] >> sh) & 0xFFu, (w[3] >> sh) & 0xFFu),
               lut_pair(lut, (w[4] >> sh) & 0xFFu, (w[5] >> sh) & 0xFFu),
               lut_pair(lut, (w[6] >> sh) & 0xFFu, (w[7] >> sh) & 0xFFu)};
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

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return uint32_t(float_to_bf16_bits(lo)) | (uint32_t(float_to_bf16_bits(hi)) << 16);
}

// MFMA mapping (v_mfma_f32_16x16x32: A row = lane % 16, B column = lane % 16,
// k-slots 8 * (lane / 16) + j; D[i][j] in lane (i / 4) * 16 + j, element i % 4):
//   S^T = K Q^T : A row = token of a 16-token block; lane group g holds dims
//                 [g * D/4, (g+1) * D/4), eight per MFMA; B column = query head.
//   O^T = V^T P': k-slot j of group g is token 4g + j (j < 4) or 16 + 4g + j - 4,
//                 which is where the S^T accumulators of the two 16-token blocks
//                 leave those tokens, so P' needs no data movement; A row r of
//                 MFMA (db, q) is dim 64 db + 4 r + q, so lane (g, n) ends up with
//                 dims 64 db + 16 g + [0, 16) of query head n contiguous.
template <int kD, bool kQBf16, bool kPaged, typename BtT>
__global__ __launch_bounds__(kThreads, 2) void paged_decode_attention_kernel(const AttnParams p) {
  constexpr int kRow = kD + 4;           // bytes per cache row
  constexpr int kLaneK = kD / 4;         // K bytes per lane per 16-token block
  constexpr int kKChunks = kD / 64;      // 16-byte K loads per lane per block
  constexpr int kQkSteps = kD / 32;      // MFMAs per 16-token block
  constexpr int kRowPieces = kD / 16;    // 16-byte pieces per V row
  constexpr int kVPieces = kD / 32;      // V pieces per lane per tile
  constexpr int kVStride = kD + 16;      // LDS bytes per staged V row (bank spread)
  constexpr int kDBlocks = kD / 64;

  __shared__ __attribute__((aligned(16))) uint16_t lut_v[256];  // bf16 payloads
  __shared__ __attribute__((aligned(16))) uint16_t lut_k[256];  // query-dtype payloads
  // Per wavefront: dec(c) * s rounded to the operand dtype for the head's K and
  // V scale s (the reference's decode_kv_rows(...).to(dtype), kv_cache.py:355-356).
  __shared__ __attribute__((aligned(16))) uint16_t lut_ks[kWaves][256];
  __shared__ __attribute__((aligned(16))) uint16_t lut_vs[kWaves][256];
  __shared__ __attribute__((aligned(16))) uint8_t vtile[kWaves][kTile * kVStride];
  __shared__ __attribute__((aligned(16))) float scl[kWaves][64];  // K scales | V scales

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  lut_v[tid] = kDeviceTables.decode_bf16[tid];
  lut_k[tid] = kQBf16 ? kDeviceTables.decode_bf16[tid] : kDeviceTables.decode_f16[tid];
  __syncthreads();  // the only workgroup barrier; waves are independent after it

  const int b = blockIdx.x / p.num_splits;
  const int split = blockIdx.x - b * p.num_splits;
  const int h = blockIdx.y * kWaves + wave;
  if (h >= p.hkv) return;
  const int len = clamp_len(p.seq_lens[b], p.max_len);
  const int n = lane & 15, g = lane >> 4;
  const bool head_ok = n < p.group;
  const int qhead = h * p.group + (head_ok ? n : 0);
  const size_t out_row = (size_t(b) * p.hq + qhead) * kD;
  const int t_begin = split * p.split_tokens;
  if (t_begin >= len) {
    if (split == 0 && head_ok) {  // empty request: zero output
      uint16_t *o = static_cast<uint16_t *>(p.out) + out_row + 16 * g;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) {
        reinterpret_cast<u32x4 *>(o + 64 * db)[0] = u32x4{0, 0, 0, 0};
        reinterpret_cast<u32x4 *>(o + 64 * db)[1] = u32x4{0, 0, 0, 0};
      }
    }
    return;
  }
  const int t_end = min(t_begin + p.split_tokens, len);
  const int ntiles = (t_end - t_begin + kTile - 1) / kTile;
  const int n_splits_b = (len + p.split_tokens - 1) / p.split_tokens;

  // Q^T operand: lane (g, n) holds dims [g*D/4, (g+1)*D/4) of query head n.
  u32x4 qf[kQkSteps];
  {
    const uint16_t *q = static_cast<const uint16_t *>(p.query) + out_row + kLaneK * g;
#pragma unroll
    for (int i = 0; i < kQkSteps; ++i)
      qf[i] = head_ok ? reinterpret_cast<const u32x4 *>(q)[i] : u32x4{0, 0, 0, 0};
  }

  const BtT *bt = static_cast<const BtT *>(p.block_table) + size_t(b) * p.bt_stride;
  const int64_t rec = int64_t(p.hkv) * kRow;  // bytes per token record
  const int64_t head_off = int64_t(h) * kRow;

  // Byte offset of row (token t, head h) and whether its block id is valid.
  // kPaged: a tile lies inside one block (block_size % 32 == 0), so the
  // lookup is per tile and tokens past the end still address that block.
  auto token_row = [&](int t, bool &ok) -> int64_t {
    const int64_t blk = int64_t(bt[t / p.block_size]);
    ok = blk >= 0 && blk < p.num_blocks;
    return ok ? (blk * p.block_size + t % p.block_size) * rec + head_off : head_off;
  };

  u32x4 kr[2][kKChunks];   // K operand bytes of the tile being computed / loaded
  u32x4 vn[kVPieces];      // next tile's V pieces
  float sn;                // next tile's K (lanes 0-31) or V (lanes 32-63) scale
  int nvalid_next;         // valid tokens of the next tile (0 if its block is invalid)
  // Rows of tokens past the end are clamped to the last valid token (generic
  // path) or stay inside the tile's block (paged path) and are masked later;
  // rows in an invalid block read the cache's first record and are masked.
  auto issue_v = [&](int t0) {
    const int nv = min(kTile, t_end - t0);
    if constexpr (kPaged) {
      bool ok;
      const int64_t base = token_row(t0, ok);
      nvalid_next = ok ? nv : 0;
#pragma unroll
      for (int j = 0; j < kVPieces; ++j) {
        const int piece = lane + 64 * j;
        const int tok = piece / kRowPieces, col = piece % kRowPieces;
        vn[j] = *reinterpret_cast<const u32x4_a4 *>(p.value_cache + base + tok * rec + 16 * col);
      }
      sn = *reinterpret_cast<const float *>((lane < 32 ? p.key_cache : p.value_cache) + base +
                                            (lane & 31) * rec + kD);
    } else {
      nvalid_next = nv;
      const int last = t_end - 1;
#pragma unroll
      for (int j = 0; j < kVPieces; ++j) {
        const int piece = lane + 64 * j;
        const int tok = piece / kRowPieces, col = piece % kRowPieces;
        bool ok;
        const int64_t off = token_row(min(t0 + tok, last), ok);
        vn[j] = ok ? *reinterpret_cast<const u32x4_a4 *>(p.value_cache + off + 16 * col) : u32x4{0, 0, 0, 0};
      }
      bool ok;
      const int64_t off = token_row(min(t0 + (lane & 31), last), ok);
      const float v = *reinterpret_cast<const float *>((lane < 32 ? p.key_cache : p.value_cache) + off + kD);
      // An invalid block's tokens get a NaN marker here and are masked.
      sn = ok ? v : __builtin_nanf("");
    }
  };
  auto issue_k = [&](int t0) {
    if constexpr (kPaged) {
      bool ok;
      const int64_t base = token_row(t0, ok);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint8_t *src = p.key_cache + base + (16 * s + n) * rec + kLaneK * g;
#pragma unroll
        for (int c = 0; c < kKChunks; ++c) kr[s][c] = *reinterpret_cast<const u32x4_a4 *>(src + 16 * c);
      }
    } else {
      const int last = t_end - 1;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        bool ok;
        const int64_t off = token_row(min(t0 + 16 * s + n, last), ok);
        const uint8_t *src = p.key_cache + off + kLaneK * g;
#pragma unroll
        for (int c = 0; c < kKChunks; ++c) kr[s][c] = *reinterpret_cast<const u32x4_a4 *>(src + 16 * c);
      }
    }
  };

  f32x4_t oacc[kDBlocks][4];
#pragma unroll
  for (int db = 0; db < kDBlocks; ++db)
#pragma unroll
    for (int q = 0; q < 4; ++q) oacc[db][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), l = 0.f;

  uint8_t *vt = vtile[wave];
  float *sc = scl[wave];
  issue_k(t_begin);
  issue_v(t_begin);
  // Scaled tables for the scales of the range's first token.  A tile whose
  // rows all carry these scales (every tile of a cache written with static
  // per-head scales) decodes K and V rounded exactly like the reference, with
  // unit per-token factors; any other tile uses the plain tables and applies
  // the row scales to the logits (K) and the softmax weights (V) in FP32.
  const float k_lut_scale = __shfl(sn, 0, kWave), v_lut_scale = __shfl(sn, 32, kWave);
  uint16_t *lks = lut_ks[wave], *lvs = lut_vs[wave];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = lane + 64 * i;
    const float v = __uint_as_float(kDeviceTables.decode_f32[c]);
    lks[c] = float_to_half_bits<kQBf16>(v * k_lut_scale);
    lvs[c] = float_to_bf16_bits(v * v_lut_scale);
  }
  for (int it = 0; it < ntiles; ++it) {
    const int t0 = t_begin + it * kTile;
    const int nvalid = nvalid_next;
    // Stage V and the scales; masked tokens get zero codes and a zero scale.
#pragma unroll
    for (int j = 0; j < kVPieces; ++j) {
      const int piece = lane + 64 * j;
      const int tok = piece / kRowPieces, col = piece % kRowPieces;
      *reinterpret_cast<u32x4 *>(vt + tok * kVStride + 16 * col) = tok < nvalid ? vn[j] : u32x4{0, 0, 0, 0};
    }
    // In the generic path a NaN scale marks an invalid block (masked too).
    const bool valid = (lane & 31) < nvalid && !__builtin_isnan(sn);
    const bool scaled = __all(!valid || sn == (lane < 32 ? k_lut_scale : v_lut_scale));
    sc[lane] = valid ? (scaled ? 1.f : sn) : 0.f;
    const uint16_t *lk = scaled ? lks : lut_k;
    const uint16_t *lv = scaled ? lvs : lut_v;
    const bool more = it + 1 < ntiles;
    if (more) issue_v(t0 + kTile);

    // S^T = K Q^T for the two 16-token blocks.
    f32x4_t sacc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      sacc[s] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < kQkSteps; ++i) {
        const u32x4 w = kr[s][i >> 1];
        const u32x4 a = (i & 1) ? decode8(lk, w[2], w[3]) : decode8(lk, w[0], w[1]);
        sacc[s] = mfma16<kQBf16>(a, qf[i], sacc[s]);
      }
    }

    if (more) issue_k(t0 + kTile);  // in flight during softmax and P V

    // Online softmax over this tile (base 2).  Lane (g, n) holds tokens
    // 4g + e and 16 + 4g + e of query head n.
    const f32x4_t ks0 = *reinterpret_cast<const f32x4_t *>(sc + 4 * g);
    const f32x4_t ks1 = *reinterpret_cast<const f32x4_t *>(sc + 16 + 4 * g);
    const f32x4_t vs0 = *reinterpret_cast<const f32x4_t *>(sc + 32 + 4 * g);
    const f32x4_t vs1 = *reinterpret_cast<const f32x4_t *>(sc + 48 + 4 * g);
    float x[8];
    float tmax = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool v0 = 4 * g + e < nvalid && ks0[e] != 0.f;
      const bool v1 = 16 + 4 * g + e < nvalid && ks1[e] != 0.f;
      x[e] = v0 ? sacc[0][e] * ks0[e] * p.scale_log2 : -__builtin_inff();
      x[4 + e] = v1 ? sacc[1][e] * ks1[e] * p.scale_log2 : -__builtin_inff();
      tmax = fmaxf(tmax, fmaxf(x[e], x[4 + e]));
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    const float m_new = fmaxf(m, tmax);
    const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    float pw[8], psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pw[e] = __builtin_amdgcn_exp2f(x[e] - m_use);
      psum += pw[e];
    }
    l = l * alpha + psum;
    m = m_new;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db)
#pragma unroll
      for (int q = 0; q < 4; ++q) oacc[db][q] *= alpha;
    const u32x4 pb{pack_bf16(pw[0] * vs0[0], pw[1] * vs0[1]), pack_bf16(pw[2] * vs0[2], pw[3] * vs0[3]),
                   pack_bf16(pw[4] * vs1[0], pw[5] * vs1[1]), pack_bf16(pw[6] * vs1[2], pw[7] * vs1[3])};

    // O^T += V^T P'.
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
      uint32_t w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tl = j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4);
        w[j] = *reinterpret_cast<const uint32_t *>(vt + tl * kVStride + 64 * db + 4 * n);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) oacc[db][q] = mfma16<true>(decode_column(lv, w, q), pb, oacc[db][q]);
    }
  }

  float lt = l + __shfl_xor(l, 16, kWave);
  lt += __shfl_xor(lt, 32, kWave);
  if (!head_ok) return;
  if (n_splits_b == 1) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t *o = static_cast<uint16_t *>(p.out) + out_row + 16 * g;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
      uint32_t packed[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        // Contiguous dim 2i (and 2i + 1) of this lane's 16 is element
        // (2i) / 4 of accumulator (2i) % 4.
        const int d0 = 2 * i, d1 = 2 * i + 1;
        const float y0 = oacc[db][d0 & 3][d0 >> 2] * inv, y1 = oacc[db][d1 & 3][d1 >> 2] * inv;
        packed[i] = uint32_t(float_to_half_bits<kQBf16>(y0)) | (uint32_t(float_to_half_bits<kQBf16>(y1)) << 16);
      }
      reinterpret_cast<u32x4 *>(o + 64 * db)[0] = u32x4{packed[0], packed[1], packed[2], packed[3]};
      reinterpret_cast<u32x4 *>(o + 64 * db)[1] = u32x4{packed[4], packed[5], packed[6], packed[7]};
    }
  } else {
    const size_t part = (size_t(b) * p.num_splits + split) * p.hq + qhead;
    float *po = p.part_o + part * kD + 16 * g;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // dims 4i .. 4i+3 of this lane's 16: element i of accumulators 0..3
        reinterpret_cast<f32x4_t *>(po + 64 * db)[i] =
            f32x4_t{oacc[db][0][i], oacc[db][1][i], oacc[db][2][i], oacc[db][3][i]};
      }
    }
    if (g == 0) {
      p.part_ml[2 * part] = m;
      p.part_ml[2 * part + 1] = lt;
    }
  }
}

// Merges the splits of each (request, query head):
//   M = max_s m_s, w_s = 2^(m_s - M), out = sum_s w_s O_s / sum_s w_s l_s.
template <bool kBf16>
__global__ __launch_bounds__(kThreads) void attention_combine_kernel(const AttnParams p) {
  __shared__ float w[kMaxSplits];
  __shared__ float red[kThreads / kWave];
  const int b = blockIdx.x / p.hq, head = blockIdx.x - b * p.hq;
  const int len = clamp_len(p.seq_lens[b], p.max_len);
  const int ns = (len + p.split_tokens - 1) / p.split_tokens;
  if (ns <= 1) return;  // written by the split kernel
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t base = size_t(b) * p.num_splits * p.hq + head;  // part index of split 0

  float mx = -__builtin_inff();
  for (int s = tid; s < ns; s += kThreads) mx = fmaxf(mx, p.part_ml[2 * (base + size_t(s) * p.hq)]);
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float lsum = 0.f;
  for (int s = tid; s < ns; s += kThreads) {
    const float ms = p.part_ml[2 * (base + size_t(s) * p.hq)];
    const float ws = ms == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
    w[s] = ws;
    lsum += ws * p.part_ml[2 * (base + size_t(s) * p.hq) + 1];
  }
  lsum = wave_sum(lsum);
  if (lane == 0) red[wave] = lsum;
  __syncthreads();
  const float total = red[0] + red[1] + red[2] + red[3];
  const float inv = total > 0.f ? 1.f / total : 0.f;
  uint16_t *o = static_cast<uint16_t *>(p.out) + (size_t(b) * p.hq + head) * p.dv;
  for (int dim = tid; dim < p.dv; dim += kThreads) {
    float acc = 0.f;
    const float *po = p.part_o + base * p.dv + dim;
    for (int s = 0; s < ns; ++s) acc += w[s] * po[size_t(s) * p.hq * p.dv];
    o[dim] = float_to_half_bits<kBf16>(acc * inv);
  }
}

// Any head size / group / block size: one wavefront per (request, query head),
// one token at a time.  Used for shapes outside the MFMA kernel's template set.
template <bool kQBf16, typename BtT>
__global__ __launch_bounds__(kWave) void paged_decode_attention_simple(const AttnParams p) {
  const int b = blockIdx.x / p.hq, head = blockIdx.x - b * p.hq;
  const int h = head / p.group;
  const int lane = threadIdx.x;
  const int len = clamp_len(p.seq_lens[b], p.max_len);
  const uint16_t *q = static_cast<const uint16_t *>(p.query) + (size_t(b) * p.hq + head) * p.d;
  const BtT *bt = static_cast<const BtT *>(p.block_table) + size_t(b) * p.bt_stride;
  const int64_t krow = p.d + 4, vrow = p.dv + 4;
  constexpr int kMaxPerLane = 8;  // head sizes up to 512
  float qv[kMaxPerLane], acc[kMaxPerLane];
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int dim = lane + kWave * i;
    qv[i] = dim < p.d ? half_bits_to_float<kQBf16>(q[dim]) : 0.f;
    acc[i] = 0.f;
  }
  float m = -__builtin_inff(), l = 0.f;
  for (int t = 0; t < len; ++t) {
    const int64_t blk = int64_t(bt[t / p.block_size]);
    if (blk < 0 || blk >= p.num_blocks) continue;
    const int64_t slot = blk * p.block_size + t % p.block_size;
    const uint8_t *kr = p.key_cache + (slot * p.hkv + h) * krow;
    const uint8_t *vr = p.value_cache + (slot * p.hkv + h) * vrow;
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      const int dim = lane + kWave * i;
      if (dim < p.d) dot = fmaf(qv[i], __uint_as_float(kDeviceTables.decode_f32[kr[dim]]), dot);
    }
    dot = wave_sum(dot);
    const float x = dot * *reinterpret_cast<const float *>(kr + p.d) * p.scale_log2;
    const float m_new = fmaxf(m, x);
    const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    const float pw = __builtin_amdgcn_exp2f(x - m_use);
    l = l * alpha + pw;
    m = m_new;
    const float pv = pw * *reinterpret_cast<const float *>(vr + p.dv);
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      const int dim = lane + kWave * i;
      acc[i] *= alpha;
      if (dim < p.dv) acc[i] = fmaf(pv, __uint_as_float(kDeviceTables.decode_f32[vr[dim]]), acc[i]);
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  uint16_t *o = static_cast<uint16_t *>(p.out) + (size_t(b) * p.hq + head) * p.dv;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int dim = lane + kWave * i;
    if (dim < p.dv) o[dim] = float_to_half_bits<kQBf16>(acc[i] * inv);
  }
}

// ------------------------------------------------------------- host side

struct SplitPlan {
  int split_tokens;
  int num_splits;
};

int env_int(const char *name, int fallback) {
  const char *v = getenv(name);
  if (!v || !*v) return fallback;
  const int x = atoi(v);
  return x > 0 ? x : fallback;
}

// Splits a request's context so that about two workgroups per CU are in
// flight over the batch (256 CUs), in whole 32-token tiles.
SplitPlan plan_splits(int64_t batch, int64_t hkv, int64_t max_len) {
  const int64_t tiles = max_len > 0 ? (max_len + kTile - 1) / kTile : 1;
  const int64_t head_groups = (hkv + kWaves - 1) / kWaves;
  const int64_t wanted = 512 / (batch * head_groups);
  const int64_t per_req = wanted < 1 ? 1 : wanted;
  int64_t tiles_per_split = (tiles + per_req - 1) / per_req;
  static const int forced = env_int("HIF8_ATTN_SPLIT_TILES", 0);
  if (forced > 0) tiles_per_split = forced;
  if (tiles_per_split < 1) tiles_per_split = 1;
  while ((tiles + tiles_per_split - 1) / tiles_per_split > kMaxSplits) tiles_per_split *= 2;
  SplitPlan plan;
  plan.split_tokens = int(tiles_per_split * kTile);
  plan.num_splits = int((tiles + tiles_per_split - 1) / tiles_per_split);
  return plan;
}

bool mfma_path(int64_t d, int64_t dv, int64_t group, int64_t block_size, const void *query, const void *out) {
  return (d == 64 || d == 128 || d == 256) && dv == d && group <= 16 && aligned(query, 16) &&
         aligned(out, 16) && block_size > 0;
}

template <int kD, bool kQBf16, typename BtT>
void launch_mfma(const AttnParams &p, int64_t batch, hipStream_t stream) {
  const dim3 grid(unsigned(batch * p.num_splits), unsigned((p.hkv + kWaves - 1) / kWaves)), block(kThreads);
  if (p.block_size % kTile == 0) paged_decode_attention_kernel<kD, kQBf16, true, BtT><<<grid, block, 0, stream>>>(p);
  else paged_decode_attention_kernel<kD, kQBf16, false, BtT><<<grid, block, 0, stream>>>(p);
  if (p.num_splits > 1) attention_combine_kernel<kQBf16><<<unsigned(batch * p.hq), kThreads, 0, stream>>>(p);
}

template <bool kQBf16, typename BtT>
void launch_attention(const AttnParams &p, bool mfma, int64_t batch, hipStream_t stream) {
  if (!mfma) {
    paged_decode_attention_simple<kQBf16, BtT><<<unsigned(batch * p.hq), kWave, 0, stream>>>(p);
    return;
  }
  switch (p.d) {
    case 64: launch_mfma<64, kQBf16, BtT>(p, batch, stream); break;
    case 128: launch_mfma<128, kQBf16, BtT>(p, batch, stream); break;
    default: launch_mfma<256, kQBf16, BtT>(p, batch, stream); break;
  }
}

}  // namespace
}  // namespace hif8

using namespace hif8;

extern "C" int hif8_kv_cache_write(const void *key, const void *value, int x_dtype, int64_t tokens,
                                   int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
                                   const float *key_scale, const float *value_scale,
                                   const void *slot_mapping, int slot_dtype, uint8_t *key_cache,
                                   uint8_t *value_cache, int64_t num_blocks, int64_t block_size,
                                   int32_t *invalid_slots, hif8_stream_t stream) {
  clear_error();
  if (tokens < 0 || num_kv_heads <= 0 || head_size <= 0 || head_size_v <= 0 || num_blocks <= 0 ||
      block_size <= 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_kv_cache_write: dimensions must be positive");
  if (head_size % 4 || head_size_v % 4)
    return fail(HIF8_ERR_INVALID_ARGUMENT,
                "hif8_kv_cache_write: head sizes must be divisible by four so the inline FP32 scale is aligned");
  if (!is_io_dtype(x_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_kv_cache_write: key/value must be float16 or bfloat16");
  if (slot_dtype != HIF8_INDEX_INT32 && slot_dtype != HIF8_INDEX_INT64)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_kv_cache_write: slot_mapping must be int32 or int64");
  if (tokens == 0) return HIF8_OK;
  if (!key || !value || !key_scale || !value_scale || !slot_mapping || !key_cache || !value_cache)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_kv_cache_write: null pointer argument");
  if (tokens > 0x7FFFFFFFll || num_kv_heads * (head_size + head_size_v) > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_kv_cache_write: dimensions too large");
  if (!aligned(key_cache, 4) || !aligned(value_cache, 4))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_kv_cache_write: caches must be 4-byte aligned");
  const uint64_t capacity = uint64_t(num_blocks) * uint64_t(block_size);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf16 = x_dtype == HIF8_DTYPE_BF16, i64 = slot_dtype == HIF8_INDEX_INT64;
  const uint16_t *k = static_cast<const uint16_t *>(key), *v = static_cast<const uint16_t *>(value);
  const uint32_t t = uint32_t(tokens), hk = uint32_t(num_kv_heads), d = uint32_t(head_size),
                 dv = uint32_t(head_size_v);
  const bool vec = head_size % 16 == 0 && head_size_v % 16 == 0 && aligned(key, 16) && aligned(value, 16);
#define HIF8_KV_WRITE(KERNEL, ITEMS)                                                                      \
  do {                                                                                                    \
    const dim3 grid(grid_for(ITEMS, 8)), block(kThreads);                                                 \
    if (bf16 && i64)                                                                                      \
      KERNEL<true, int64_t><<<grid, block, 0, s>>>(k, v, key_scale, value_scale,                          \
                                                   static_cast<const int64_t *>(slot_mapping), key_cache, \
                                                   value_cache, t, hk, d, dv, capacity, invalid_slots);   \
    else if (bf16)                                                                                        \
      KERNEL<true, int32_t><<<grid, block, 0, s>>>(k, v, key_scale, value_scale,                          \
                                                   static_cast<const int32_t *>(slot_mapping), key_cache, \
                                                   value_cache, t, hk, d, dv, capacity, invalid_slots);   \
    else if (i64)                                                                                         \
      KERNEL<false, int64_t><<<grid, block, 0, s>>>(k, v, key_scale, value_scale,                         \
                                                    static_cast<const int64_t *>(slot_mapping), key_cache,\
                                                    value_cache, t, hk, d, dv, capacity, invalid_slots);  \
    else                                                                                                  \
      KERNEL<false, int32_t><<<grid, block, 0, s>>>(k, v, key_scale, value_scale,                         \
                                                    static_cast<const int32_t *>(slot_mapping), key_cache,\
                                                    value_cache, t, hk, d, dv, capacity, invalid_slots);  \
  } while (0)
  if (vec) HIF8_KV_WRITE(kv_write_vec16, uint64_t(tokens) * num_kv_heads * (head_size + head_size_v) / 16);
  else HIF8_KV_WRITE(kv_write_scalar, uint64_t(tokens) * num_kv_heads * (head_size + head_size_v));
#undef HIF8_KV_WRITE
  return check_launch("hif8_kv_cache_write");
}

extern "C" size_t hif8_paged_decode_attention_workspace_size(int64_t batch, int64_t num_heads,
                                                             int64_t num_kv_heads, int64_t head_size,
                                                             int64_t head_size_v, int64_t max_seq_len) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 || head_size_v <= 0 ||
      max_seq_len <= 0 || num_heads % num_kv_heads)
    return 0;
  if (!((head_size == 64 || head_size == 128 || head_size == 256) && head_size_v == head_size &&
        num_heads / num_kv_heads <= 16))
    return 0;  // the one-wavefront-per-head kernel needs no workspace
  const SplitPlan plan = plan_splits(batch, num_kv_heads, max_seq_len);
  if (plan.num_splits <= 1) return 0;
  return size_t(batch) * size_t(plan.num_splits) * size_t(num_heads) * size_t(head_size_v + 2) * sizeof(float);
}

extern "C" int hif8_paged_decode_attention(const void *query, int q_dtype, const uint8_t *key_cache,
                                           const uint8_t *value_cache, int64_t num_blocks, int64_t block_size,
                                           int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
                                           const void *block_table, int block_table_dtype,
                                           int64_t max_blocks_per_seq, const int32_t *seq_lens, int64_t batch,
                                           int64_t num_heads, int64_t max_seq_len, float scale, void *out,
                                           void *workspace, size_t workspace_bytes, hif8_stream_t stream) {
  clear_error();
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 || head_size_v <= 0 ||
      num_blocks <= 0 || block_size <= 0 || max_blocks_per_seq <= 0 || max_seq_len < 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: dimensions must be positive");
  if (num_heads % num_kv_heads)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: num_heads must be divisible by num_kv_heads");
  if (head_size % 4 || head_size_v % 4)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: head sizes must be divisible by four");
  if (head_size > 512 || head_size_v > 512)
    return fail(HIF8_ERR_UNSUPPORTED, "hif8_paged_decode_attention: head sizes above 512 are not supported");
  if (!is_io_dtype(q_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: query must be float16 or bfloat16");
  if (block_table_dtype != HIF8_INDEX_INT32 && block_table_dtype != HIF8_INDEX_INT64)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: block_table must be int32 or int64");
  if (max_seq_len > max_blocks_per_seq * block_size)
    return fail(HIF8_ERR_INVALID_ARGUMENT,
                "hif8_paged_decode_attention: max_seq_len exceeds the block table capacity");
  if (max_seq_len > 0x7FFFFFFFll || batch > 0x7FFFFFFFll || num_heads > 0xFFFF)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: dimensions too large");
  if (batch == 0) return HIF8_OK;
  if (!query || !key_cache || !value_cache || !block_table || !seq_lens || !out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: null pointer argument");
  if (!aligned(key_cache, 4) || !aligned(value_cache, 4))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: caches must be 4-byte aligned");
  if (!aligned(query, 2) || !aligned(out, 2))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: query/out must be 2-byte aligned");

  AttnParams p{};
  p.query = query;
  p.key_cache = key_cache;
  p.value_cache = value_cache;
  p.block_table = block_table;
  p.seq_lens = seq_lens;
  p.out = out;
  p.bt_stride = max_blocks_per_seq;
  p.num_blocks = num_blocks;
  p.block_size = int(block_size);
  p.hkv = int(num_kv_heads);
  p.hq = int(num_heads);
  p.group = int(num_heads / num_kv_heads);
  p.d = int(head_size);
  p.dv = int(head_size_v);
  p.max_len = int(max_seq_len);
  p.scale_log2 = scale * 1.4426950408889634f;
  const bool mfma = mfma_path(head_size, head_size_v, p.group, block_size, query, out);
  if (mfma) {
    const SplitPlan plan = plan_splits(batch, num_kv_heads, max_seq_len);
    p.split_tokens = plan.split_tokens;
    p.num_splits = plan.num_splits;
    if (plan.num_splits > 1) {
      const size_t need = hif8_paged_decode_attention_workspace_size(batch, num_heads, num_kv_heads, head_size,
                                                                     head_size_v, max_seq_len);
      if (!workspace || workspace_bytes < need)
        return fail(HIF8_ERR_INVALID_ARGUMENT,
                    "hif8_paged_decode_attention: workspace of %zu bytes required (got %zu)", need,
                    workspace_bytes);
      if (!aligned(workspace, 16))
        return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_paged_decode_attention: workspace must be 16-byte aligned");
      p.part_o = static_cast<float *>(workspace);
      p.part_ml = p.part_o + size_t(batch) * plan.num_splits * num_heads * head_size_v;
    }
  } else {
    p.split_tokens = p.max_len > 0 ? p.max_len : 1;
    p.num_splits = 1;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool bf16 = q_dtype == HIF8_DTYPE_BF16, i64 = block_table_dtype == HIF8_INDEX_INT64;
  if (bf16 && i64) launch_attention<true, int64_t>(p, mfma, batch, s);
  else if (bf16) launch_attention<true, int32_t>(p, mfma, batch, s);
  else if (i64) launch_attention<false, int64_t>(p, mfma, batch, s);
  else launch_attention<false, int32_t>(p, mfma, batch, s);
  return check_launch("hif8_paged_decode_attention");
}
