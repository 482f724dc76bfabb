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
// (request, token range = "split", KV head) and has D / 64 wavefronts, one
// per 64-dim slice of K and V (so a tile's decode work is spread over the
// SIMDs); the block ids of the KV heads of one split are adjacent modulo 8, so
// they run on one XCD and share its L2.  The workgroup walks its range in
// 32-token tiles:
//   * K slices go from HBM straight into VGPRs in the MFMA A-operand layout
//     (token = lane % 16, 16 contiguous bytes per lane) and each wavefront's
//     share of S^T = K Q^T runs on v_mfma_f32_16x16x32 (B = the G query heads
//     of the KV head, padded to 16 columns); the shares are summed through
//     LDS in wavefront order, so every wavefront runs the same softmax;
//   * V slices are copied raw into LDS by DMA (global_load_lds_dwordx4) and
//     read transposed (8 tokens x 4 dims per lane), and O^T += V^T P' runs on
//     the same MFMA with the softmax weights P' rounded to the query dtype;
//   * both operands are decoded through per-wave LDS tables that hold
//     dtype(dec(c) * s) for the tile's row scale s - which is how the
//     reference decodes K and V before its attention
//     (decode_kv_rows(...).to(query dtype), kv_cache.py:355-356); static
//     caches give every row of a head the same scale, so a table is rebuilt
//     only when the scale changes.  A tile whose rows mix scales uses the
//     exact decode (s = 1) and applies the FP32 row scales to the scores and
//     the softmax weights instead (equal up to rounding);
//   * the online softmax keeps (max, sum) per query head in FP32;
//   * the next tile's loads are in flight while the current tile computes.
// HiF8 values are exact in bf16 and fp16, so decode adds no rounding.  With
// more than one split per request, partial (O, max, sum) go to the caller's
// workspace and a second kernel merges them.
#include <stddef.h>
#include <stdlib.h>

#include <mutex>
#include <type_traits>

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
    // Non-temporal stores: the pages are read by a later step's attention,
    // not by this one (4096 tokens: 9.5 -> 9.0 us on MI355X).
    __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]}, reinterpret_cast<u32x4_a4 *>(row + 16 * col));
    if (col == 0) __builtin_nontemporal_store(s, reinterpret_cast<float *>(row + width));
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
  int block_size, log2_block_size, hkv, hq, group, d, dv;
  int max_len, split_tokens, num_splits, batch;
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

// Two fp32 values rounded to nearest-even and packed as the MFMA operand dtype.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <bool kBf16>
__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
  if constexpr (kBf16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
  } else {
    return uint32_t(float_to_f16_bits(lo)) | (uint32_t(float_to_f16_bits(hi)) << 16);
  }
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


// MFMA mapping (v_mfma_f32_16x16x32: A row = lane % 16, B column = lane % 16,
// k-slots 8 * (lane / 16) + j; D[i][j] in lane (i / 4) * 16 + j, element i % 4).
// A workgroup has D / 64 wavefronts; wavefront w owns dims [64 w, 64 w + 64)
// of K and V, so each one decodes a quarter of the codes of a D = 256 tile:
//   S^T = K Q^T : A row = token of a 16-token block; lane group g holds the
//                 16 dims 64 w + 16 g + [0, 16) (two MFMAs of 8 k-slots), one
//                 16-byte load per lane; B column = query head.  The partial
//                 scores of the wavefronts are summed through LDS in wavefront
//                 order, so every wavefront holds the same S and runs the same
//                 online softmax.
//   O^T = V^T P': k-slot j of group g is token 4g + j (j < 4) or 16 + 4g + j - 4,
//                 which is where the S^T accumulators of the two 16-token blocks
//                 leave those tokens, so P' needs no data movement; A row r of
//                 MFMA q is dim 64 w + 4 r + q, so lane (g, n) ends up with
//                 dims 64 w + 16 g + [0, 16) of query head n contiguous.
// Each wavefront copies the 64-byte V slice of its dims into LDS by DMA; the
// 16-byte granule c of token t lands in slot 64 (t >> 4) + 16 (t & 3) +
// 4 ((t >> 2) & 3) + c, so the transposed reads (token 4g + j for the four lane
// groups) touch 64 different banks.
//
// Workgroups of the Hkv heads of one split get block ids that are equal
// modulo 8, so they run on the same XCD and the cache lines their rows share
// are read from HBM once.
template <int kD, bool kQBf16, bool kPaged, typename BtT>
__global__ __launch_bounds__(kWave * (kD / 64), 4) void paged_decode_attention_kernel(const AttnParams p) {
  constexpr int kRow = kD + 4;            // bytes per cache row
  constexpr int kWd = kD / 64;            // wavefronts per workgroup, 64 dims each
  constexpr int kSlice = kTile * 64;      // one wavefront's V bytes of a tile
  static_assert(kTile == 32, "the V slot map and the P' layout assume 32-token tiles");
  static_assert(kD % 64 == 0 && kWd >= 1 && kWd <= 4, "64-dim slices");

  struct Smem {
    // The decode tables first (Smem is the kernel's only LDS object): at fixed
    // LDS addresses 0 and 512 a lookup address is one shift of the code byte.
    uint16_t k_tab[256];           // query dtype(dec(c) * k_tab_scale)
    uint16_t v_tab[256];           // query dtype(dec(c) * v_tab_scale) or (mixed scales) bf16(dec(c))
    float scl[kWd][64];            // K | V factors of the tile's tokens (0 = masked)
    f32x4_t sx[2][kWd][2][kWave];  // partial scores [tile parity][wavefront][16-token block][lane]
    uint8_t vtile[2][kWd][kSlice]; // double-buffered V slices
  };
  __shared__ __attribute__((aligned(16))) Smem smem;

  const int xcd = int(blockIdx.x) & 7, slot_id = int(blockIdx.x) >> 3;
  const int h = slot_id % p.hkv;
  const int bs_idx = (slot_id / p.hkv) * 8 + xcd;
  if (bs_idx >= p.batch * p.num_splits) return;  // padding block (uniform)
  const int b = bs_idx / p.num_splits;
  const int split = bs_idx - b * p.num_splits;
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int lane = int(threadIdx.x) & 63;
  const int n = lane & 15, g = lane >> 4;
  const bool head_ok = n < p.group;
  const int qhead = h * p.group + (head_ok ? n : 0);
  const size_t out_row = (size_t(b) * p.hq + qhead) * kD;
  const int t_begin = split * p.split_tokens;
  // The range end from max_len alone: the first loads need no length.
  const int t_cap = min(t_begin + p.split_tokens, p.max_len);

  const BtT *bt = static_cast<const BtT *>(p.block_table) + size_t(b) * p.bt_stride;
  const int64_t rec = int64_t(p.hkv) * kRow;  // bytes per token record
  const int64_t head_off = int64_t(h) * kRow;
  const int lg = p.log2_block_size;

  // The block ids of this split, one per lane (a split spans at most 64
  // blocks), loaded once so that no tile waits on a table load.
  const int first_blk = t_begin >> lg;
  int64_t blk_lane;
  {
    const int last_blk = (max(t_cap, t_begin + 1) - 1) >> lg;
    blk_lane = int64_t(bt[min(first_blk + lane, last_blk)]);
  }
  const bool blk_lane_ok = blk_lane >= 0 && blk_lane < p.num_blocks;
  const int64_t slot_lane = blk_lane_ok ? (blk_lane << lg) : int64_t(-1);  // first flat slot of the block

  // Byte offset of row (token t, head h) and whether its block id is valid;
  // rows in an invalid block read the cache's first record and are masked.
  // kPaged: a tile lies inside one block (block_size % 32 == 0), so the
  // lookup is per tile (a lane read) and tokens past the end still address
  // that block.
  auto tile_row = [&](int t0, bool &ok) -> int64_t {
    const int idx = (t0 >> lg) - first_blk;
    const int lo = __builtin_amdgcn_readlane(int(uint64_t(slot_lane)), idx);
    const int hi = __builtin_amdgcn_readlane(int(uint64_t(slot_lane) >> 32), idx);
    const int64_t slot0 = int64_t((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
    ok = slot0 >= 0;
    return ok ? (slot0 + (t0 & ((1 << lg) - 1))) * rec + head_off : head_off;
  };
  auto token_row = [&](int t, bool &ok) -> int64_t {
    const int idx = (t >> lg) - first_blk;
    const int lo = __shfl(int(uint64_t(slot_lane)), idx, kWave);
    const int hi = __shfl(int(uint64_t(slot_lane) >> 32), idx, kWave);
    const int64_t slot0 = int64_t((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
    ok = slot0 >= 0;
    return ok ? (slot0 + (t & ((1 << lg) - 1))) * rec + head_off : head_off;
  };

  const int dim0 = 64 * wv;  // first dim of this wavefront
  u32x4 kn[2];               // K bytes (dims dim0 + 16 g + [0, 16)) of the tile in flight
  float sn;                  // K (lanes 0-31) or V (lanes 32-63) scale of token lane % 32
  bool tile_ok_next;         // the block of the tile in flight is valid (paged path)
  const uint32_t vbuf_lds = __builtin_amdgcn_readfirstlane(lds_address(&smem.vtile[0][wv][0]));
  // DMA lane -> token of the V slot map: lane i of copy j fills slot 64 j + i.
  const int dma_tok = 4 * ((lane >> 2) & 3) + (lane >> 4);
  // Loads of tile t0 whose tokens end at t_last: V by DMA into buffer `buf`,
  // scales into sn, K into kn.  Tokens past t_last address t_last (generic
  // path) or stay inside the tile's block (paged path); they are masked later.
  auto issue = [&](int t0, int t_last, int buf) {
    const uint32_t dst = vbuf_lds + uint32_t(buf * kWd * kSlice);
    if constexpr (kPaged) {
      bool ok;
      const int64_t base = tile_row(t0, ok);
      tile_ok_next = ok;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        dma16(p.value_cache + base + (16 * j + dma_tok) * rec + dim0 + 16 * (lane & 3), dst + 1024u * j);
#pragma unroll
      for (int s = 0; s < 2; ++s)
        kn[s] = *reinterpret_cast<const u32x4_a4 *>(p.key_cache + base + (16 * s + n) * rec + dim0 + 16 * g);
      sn = *reinterpret_cast<const float *>((lane < 32 ? p.key_cache : p.value_cache) + base +
                                            (lane & 31) * rec + kD);
    } else {
      tile_ok_next = true;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bool ok;
        const int64_t off = token_row(min(t0 + 16 * j + dma_tok, t_last), ok);
        dma16(p.value_cache + off + dim0 + 16 * (lane & 3), dst + 1024u * j);
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        bool ok;
        const int64_t off = token_row(min(t0 + 16 * s + n, t_last), ok);
        kn[s] = *reinterpret_cast<const u32x4_a4 *>(p.key_cache + off + dim0 + 16 * g);
      }
      bool ok;
      const int64_t off = token_row(min(t0 + (lane & 31), t_last), ok);
      const float v = *reinterpret_cast<const float *>((lane < 32 ? p.key_cache : p.value_cache) + off + kD);
      sn = ok ? v : 0.f;  // a zero scale masks the token
    }
  };

  // Prologue, independent of the request length: the first tile, the
  // query, the fp32 decode table.
  const int len_raw = p.seq_lens[b];
  issue(t_begin, t_cap - 1, 0);
  u32x4 qf[2];
  {
    // Q^T operand: lane (g, n) holds dims dim0 + 16 g + [0, 16) of query head n.
    const u32x4 *q = reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(p.query) + out_row + dim0 + 16 * g);
    qf[0] = head_ok ? q[0] : u32x4{0, 0, 0, 0};
    qf[1] = head_ok ? q[1] : u32x4{0, 0, 0, 0};
  }
  // Each wavefront writes a quarter of the shared tables (entries 64 wv + lane;
  // a D = 128 / D = 64 workgroup's wavefronts write two / four quarters each).
  float decf[4 / kWd];
#pragma unroll
  for (int i = 0; i < 4 / kWd; ++i) decf[i] = __uint_as_float(kDeviceTables.decode_f32[lane + 64 * (wv + kWd * i)]);
  // The scales the tables currently hold (NaN: not built yet).
  float k_tab_scale = __builtin_nanf(""), v_tab_scale = __builtin_nanf("");

  const int len = clamp_len(len_raw, p.max_len);
  if (t_begin >= len) {  // an empty split
    wait_vmcnt<0>();     // no copy may still target LDS when the wave ends
    if (split == 0) {    // an empty request: zero output
      uint16_t *o = static_cast<uint16_t *>(p.out) + (size_t(b) * p.hq + h * p.group) * kD + dim0;
      for (int i = lane; i < p.group * 64; i += kWave) o[(i >> 6) * kD + (i & 63)] = 0;
    }
    return;
  }
  const int t_end = min(t_cap, len);
  const int n_splits_b = (len + p.split_tokens - 1) / p.split_tokens;
  const int ntiles = (t_end - t_begin + kTile - 1) / kTile;

  f32x4_t oacc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) oacc[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), l = 0.f;
  float *sc = smem.scl[wv];
  const uint16_t *kl = smem.k_tab;
  const uint16_t *vl = smem.v_tab;

  for (int it = 0; it < ntiles; ++it) {
    const int t0 = t_begin + it * kTile;
    const int nvalid = min(kTile, t_end - t0);
    wait_vmcnt<0>();
    const float s_cur = sn;
    const bool blk_ok = tile_ok_next;
    const u32x4 kc[2] = {kn[0], kn[1]};
    uint8_t *vt = &smem.vtile[it & 1][wv][0];
    // The next tile is in flight during this one.
    if (it + 1 < ntiles) issue(t0 + kTile, t_end - 1, (it + 1) & 1);

    // A block id outside the cache masks the whole tile.
    const bool valid = blk_ok && (lane & 31) < nvalid && s_cur != 0.f;
    // When the valid K rows (lanes 0-31) or V rows (lanes 32-63) of the tile
    // share one scale (always, for a cache written with static per-head
    // scales), that table holds dtype(dec(c) * scale) - the values the
    // reference decodes K/V to (kv_cache.py:355-356) - and the rows get unit
    // factors; otherwise it holds the exact dec(c) and the row scales multiply
    // the logits (K) and softmax weights (V) in FP32.
    const uint64_t vball = __ballot(valid);
    const int k_first = __builtin_ffsll(vball & 0xFFFFFFFFull) - 1;
    const int v_first = __builtin_ffsll(vball & 0xFFFFFFFF00000000ull) - 1;
    const float k_one = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s_cur), max(k_first, 0)));
    const float v_one = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s_cur), max(v_first, 32)));
    const uint64_t same = __ballot(!valid || s_cur == (lane < 32 ? k_one : v_one));
    const bool k_uniform = (same & 0xFFFFFFFFull) == 0xFFFFFFFFull;
    const bool v_uniform = (same >> 32) == 0xFFFFFFFFull;
    const float k_want = k_uniform ? k_one : 1.f, v_want = v_uniform ? v_one : 1.f;
    // V and P' go through the MFMA in the query dtype when the tile's V rows
    // share a scale (the reference rounds V and the softmax weights to
    // query.dtype, kv_cache.py:355-356 and :370-371); with mixed scales the
    // table holds the exact dec(c) in bf16 and P' = P * row scale stays bf16
    // (fp16 would lose P' * scale below 2^-14 to subnormals).  The sentinel
    // -1 marks the exact bf16 table of an fp16-query kernel.
    const float v_key = kQBf16 || v_uniform ? v_want : -1.f;
    // The tables are shared by the workgroup's wavefronts, which all see the
    // same tile scales: a rebuild (once per workgroup for a cache with static
    // per-head scales) waits until every wavefront is done with the old
    // tables, and the lookups wait until every quarter is written.
    const bool k_new = !(k_want == k_tab_scale), v_new = !(v_key == v_tab_scale);
    if (k_new || v_new) {
      if (it > 0) lds_barrier();
#pragma unroll
      for (int i = 0; i < 4 / kWd; ++i) {
        const int e = lane + 64 * (wv + kWd * i);
        if (k_new) smem.k_tab[e] = float_to_half_bits<kQBf16>(decf[i] * k_want);
        if (v_new)
          smem.v_tab[e] =
              v_uniform ? float_to_half_bits<kQBf16>(decf[i] * v_want) : float_to_bf16_bits(decf[i] * v_want);
      }
      k_tab_scale = k_want;
      v_tab_scale = v_key;
      lds_barrier();
    }
    sc[lane] = valid ? ((lane < 32 ? k_uniform : v_uniform) ? 1.f : s_cur) : 0.f;
    if (!__all(valid)) {
      // Masked tokens: zero their V codes so that 0 * Inf / NaN cannot reach O.
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int tok = 16 * j + dma_tok;
        if (!(tok < nvalid && sc[tok] != 0.f))
          *reinterpret_cast<u32x4 *>(vt + 1024 * j + 16 * lane) = u32x4{0, 0, 0, 0};
      }
    }

    // This wavefront's share of S^T = K Q^T for the two 16-token blocks.
    f32x4_t sacc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      sacc[s] = mfma16<kQBf16>(decode8(kl, kc[s][0], kc[s][1]), qf[0], f32x4_t{0.f, 0.f, 0.f, 0.f});
      sacc[s] = mfma16<kQBf16>(decode8(kl, kc[s][2], kc[s][3]), qf[1], sacc[s]);
    }
    if constexpr (kWd > 1) {
      // Sum the partial scores in wavefront order (the same in every wavefront).
      // Columns of padding heads are zero in every partial and stay unsummed.
      const int par = it & 1;
      if (head_ok) {
        smem.sx[par][wv][0][lane] = sacc[0];
        smem.sx[par][wv][1][lane] = sacc[1];
      }
      lds_barrier();
      if (head_ok) {
        f32x4_t s0 = smem.sx[par][0][0][lane], s1 = smem.sx[par][0][1][lane];
#pragma unroll
        for (int w2 = 1; w2 < kWd; ++w2) {
          s0 += smem.sx[par][w2][0][lane];
          s1 += smem.sx[par][w2][1][lane];
        }
        sacc[0] = s0;
        sacc[1] = s1;
      }
    }

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
      x[e] = ks0[e] != 0.f ? sacc[0][e] * ks0[e] * p.scale_log2 : -__builtin_inff();
      x[4 + e] = ks1[e] != 0.f ? sacc[1][e] * ks1[e] * p.scale_log2 : -__builtin_inff();
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
    // The output needs rescaling only when some head's running max moved
    // from a finite value (before that the accumulators are zero).
    if (!__all(m_new == m || m == -__builtin_inff())) {
#pragma unroll
      for (int q = 0; q < 4; ++q) oacc[q] *= alpha;
    }
    m = m_new;
    // O^T += V^T P' over this wavefront's 64 dims: word j holds dims
    // dim0 + 4n + [0, 4) of token 4g + j (j < 4) or 16 + 4g + j - 4.
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      w[j] = *reinterpret_cast<const uint32_t *>(vt + 1024 * (j >> 2) + 256 * (j & 3) + 64 * g + 4 * n);
    // P' = P * (1 for a valid row of a uniform tile, the row scale for mixed
    // tiles, 0 for a masked row).
    auto pv = [&](auto bf16_mma) {
      constexpr bool kB = decltype(bf16_mma)::value;
      const u32x4 pb{pack_half2<kB>(pw[0] * vs0[0], pw[1] * vs0[1]), pack_half2<kB>(pw[2] * vs0[2], pw[3] * vs0[3]),
                     pack_half2<kB>(pw[4] * vs1[0], pw[5] * vs1[1]), pack_half2<kB>(pw[6] * vs1[2], pw[7] * vs1[3])};
#pragma unroll
      for (int q = 0; q < 4; ++q) oacc[q] = mfma16<kB>(decode_column(vl, w, q), pb, oacc[q]);
    };
    if (kQBf16 || !v_uniform) pv(std::true_type{});
    else pv(std::false_type{});
  }
  float lt = l + __shfl_xor(l, 16, kWave);
  lt += __shfl_xor(lt, 32, kWave);
  if (!head_ok) return;
  if (n_splits_b == 1) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t *o = static_cast<uint16_t *>(p.out) + out_row + dim0 + 16 * g;
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // Contiguous dim 2i (and 2i + 1) of this lane's 16 is element
      // (2i) / 4 of accumulator (2i) % 4.
      const int d0 = 2 * i, d1 = 2 * i + 1;
      packed[i] = pack_half2<kQBf16>(oacc[d0 & 3][d0 >> 2] * inv, oacc[d1 & 3][d1 >> 2] * inv);
    }
    reinterpret_cast<u32x4 *>(o)[0] = u32x4{packed[0], packed[1], packed[2], packed[3]};
    reinterpret_cast<u32x4 *>(o)[1] = u32x4{packed[4], packed[5], packed[6], packed[7]};
  } else {
    const size_t part = (size_t(b) * p.num_splits + split) * p.hq + qhead;
    float *po = p.part_o + part * kD + dim0 + 16 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // dims 4i .. 4i+3 of this lane's 16: element i of accumulators 0..3
      reinterpret_cast<f32x4_t *>(po)[i] = f32x4_t{oacc[0][i], oacc[1][i], oacc[2][i], oacc[3][i]};
    }
    if (g == 0 && wv == 0) {
      p.part_ml[2 * part] = m;
      p.part_ml[2 * part + 1] = lt;
    }
  }
}

// Merges the splits of each (request, query head, 64-dim slice):
//   M = max_s m_s, w_s = 2^(m_s - M), out = sum_s w_s O_s / sum_s w_s l_s.
// Four groups of 64 threads take every fourth split; each thread one dim.
constexpr int kCombineDims = 16;  // output dims per combine block

template <bool kBf16>
__global__ __launch_bounds__(kThreads) void attention_combine_kernel(const AttnParams p) {
  __shared__ float w[kMaxSplits];
  __shared__ float red[kThreads];
  const int b = blockIdx.x / p.hq, head = blockIdx.x - b * p.hq;
  const int len = clamp_len(p.seq_lens[b], p.max_len);
  const int ns = (len + p.split_tokens - 1) / p.split_tokens;
  if (ns <= 1) return;  // written by the split kernel
  const int tid = threadIdx.x, lane = tid & 63, grp = tid >> 6;
  const size_t base = size_t(b) * p.num_splits * p.hq + head;  // part index of split 0
  const size_t stride = size_t(p.hq);                           // parts between splits

  float mx = -__builtin_inff();
  for (int s = tid; s < ns; s += kThreads) mx = fmaxf(mx, p.part_ml[2 * (base + s * stride)]);
  mx = wave_max(mx);
  if (lane == 0) red[grp] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float lsum = 0.f;
  for (int s = tid; s < ns; s += kThreads) {
    const float ms = p.part_ml[2 * (base + s * stride)];
    const float ws = ms == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(ms - mx);
    w[s] = ws;
    lsum += ws * p.part_ml[2 * (base + s * stride) + 1];
  }
  lsum = wave_sum(lsum);
  if (lane == 0) red[grp] = lsum;
  __syncthreads();
  const float total = red[0] + red[1] + red[2] + red[3];
  const float inv = total > 0.f ? 1.f / total : 0.f;
  __syncthreads();
  // 16 dims per block, 16 split groups: thread (d, g) sums splits s = g mod 16
  // of dim blockIdx.y * 16 + d, so every CU gets work even for one request.
  const int d = tid & 15, g = tid >> 4;
  const int dim = int(blockIdx.y) * kCombineDims + d;
  float acc = 0.f;
  if (dim < p.dv) {
    const float *po = p.part_o + base * p.dv + dim;
    const size_t sstride = stride * p.dv;
    int s = g;
    float a0 = 0.f, a1 = 0.f;
    for (; s + 16 < ns; s += 32) {
      a0 += w[s] * po[s * sstride];
      a1 += w[s + 16] * po[(s + 16) * sstride];
    }
    for (; s < ns; s += 16) a0 += w[s] * po[s * sstride];
    acc = a0 + a1;
  }
  red[tid] = acc;
  __syncthreads();
  if (tid < kCombineDims && dim < p.dv) {
    float y = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) y += red[16 * j + tid];
    static_cast<uint16_t *>(p.out)[(size_t(b) * p.hq + head) * p.dv + dim] = float_to_half_bits<kBf16>(y * inv);
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
    // K and V rows decoded to the query dtype, dtype(dec(c) * row scale)
    // (kv_cache.py:355-356), as in the MFMA kernel.
    const float ksc = *reinterpret_cast<const float *>(kr + p.d);
    const float vsc = *reinterpret_cast<const float *>(vr + p.dv);
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      const int dim = lane + kWave * i;
      if (dim < p.d)
        dot = fmaf(qv[i], half_bits_to_float<kQBf16>(float_to_half_bits<kQBf16>(
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
        acc[i] = fmaf(pw, half_bits_to_float<kQBf16>(float_to_half_bits<kQBf16>(
                              __uint_as_float(kDeviceTables.decode_f32[vr[dim]]) * vsc)), acc[i]);
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

// At most this many tiles per split: a split then spans at most 62 blocks of
// the smallest block size the MFMA kernel takes (16), one block id per lane.
constexpr int kMaxTilesPerSplit = 31;

// Splits a request's context in whole 32-token tiles: as many tiles per
// split as keep at least ~512 workgroups (two per CU, D / 64 wavefronts
// each) over the batch and the KV heads, at most 8, and enough that the
// split count fits the combine kernel.  Measured on MI355X over 1..16 tiles
// per split at B=1/4 x ctx 512..16384: B=1 ctx 16384 22.5 -> 20.6 us with 4
// tiles instead of 2, B=4 ctx 4096 21.1 -> 19.9, B=4 ctx 16384 48.3 -> 46.1
// with 8 instead of 4; one tile where the context is short.
SplitPlan plan_splits(int64_t batch, int64_t hkv, int64_t max_len) {
  const int64_t tiles = max_len > 0 ? (max_len + kTile - 1) / kTile : 1;
  int64_t per_split = (batch * hkv * tiles) / 512;
  if (per_split > 8) per_split = 8;
  const int64_t fit = (tiles + kMaxSplits - 1) / kMaxSplits;
  if (per_split < fit) per_split = fit;
  static const int forced = env_int("HIF8_ATTN_SPLIT_TILES", 0);
  if (forced > 0) per_split = forced;
  if (per_split > kMaxTilesPerSplit) per_split = kMaxTilesPerSplit;
  if (per_split < 1) per_split = 1;
  SplitPlan plan;
  plan.split_tokens = int(per_split * kTile);
  plan.num_splits = int((max_len + plan.split_tokens - 1) / plan.split_tokens);
  if (plan.num_splits < 1) plan.num_splits = 1;
  return plan;
}

bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int log2_of(int64_t v) {
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return l;
}

// Shapes the MFMA kernel takes (the rest runs the one-wavefront-per-head kernel).
bool mfma_shape(int64_t d, int64_t dv, int64_t group, int64_t block_size, int64_t max_len) {
  return (d == 64 || d == 128 || d == 256) && dv == d && group <= 16 && pow2(block_size) && block_size >= 16 &&
         max_len <= int64_t(kMaxSplits) * kMaxTilesPerSplit * kTile;
}

bool mfma_path(int64_t d, int64_t dv, int64_t group, int64_t block_size, int64_t max_len, const void *query,
               const void *out) {
  return mfma_shape(d, dv, group, block_size, max_len) && aligned(query, 16) && aligned(out, 16);
}

template <int kD, bool kQBf16, typename BtT>
void launch_mfma(const AttnParams &p, int64_t batch, hipStream_t stream) {
  // Block id = ((request split group of 8) * Hkv + head) * 8 + position in the group.
  const int64_t groups = (batch * p.num_splits + 7) / 8;
  const dim3 grid(unsigned(groups * 8 * p.hkv)), block(kWave * (kD / 64));
  if (p.block_size % kTile == 0) paged_decode_attention_kernel<kD, kQBf16, true, BtT><<<grid, block, 0, stream>>>(p);
  else paged_decode_attention_kernel<kD, kQBf16, false, BtT><<<grid, block, 0, stream>>>(p);
  if (p.num_splits > 1)
    attention_combine_kernel<kQBf16><<<dim3(unsigned(batch * p.hq), unsigned((p.dv + kCombineDims - 1) / kCombineDims)),
                                       kThreads, 0, stream>>>(p);
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
  // Any power-of-two block size >= 16 qualifies; the workspace does not depend on it.
  if (!mfma_shape(head_size, head_size_v, num_heads / num_kv_heads, 16, max_seq_len))
    return 0;  // the one-wavefront-per-head kernel needs no workspace
  const SplitPlan plan = plan_splits(batch, num_kv_heads, max_seq_len);
  if (plan.num_splits <= 1) return 0;
  return size_t(batch) * size_t(plan.num_splits) * size_t(num_heads) * size_t(head_size_v + 2) * sizeof(float);
}

namespace hif8 {
namespace {

// The decode attention of both entry points below; `name` prefixes errors.
int decode_attention(const char *name, const void *query, int q_dtype, const uint8_t *key_cache,
                     const uint8_t *value_cache, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                     int64_t head_size, int64_t head_size_v, const void *block_table, int block_table_dtype,
                     int64_t max_blocks_per_seq, const int32_t *seq_lens, int64_t batch, int64_t num_heads,
                     int64_t max_seq_len, float scale, void *out, void *workspace, size_t workspace_bytes,
                     hif8_stream_t stream) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 || head_size_v <= 0 ||
      num_blocks <= 0 || block_size <= 0 || max_blocks_per_seq <= 0 || max_seq_len < 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: dimensions must be positive", name);
  if (num_heads % num_kv_heads)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: num_heads must be divisible by num_kv_heads", name);
  if (head_size % 4 || head_size_v % 4)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: head sizes must be divisible by four", name);
  if (head_size > 512 || head_size_v > 512)
    return fail(HIF8_ERR_UNSUPPORTED, "%s: head sizes above 512 are not supported", name);
  if (!is_io_dtype(q_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: query must be float16 or bfloat16", name);
  if (block_table_dtype != HIF8_INDEX_INT32 && block_table_dtype != HIF8_INDEX_INT64)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: block_table must be int32 or int64", name);
  if (max_seq_len > max_blocks_per_seq * block_size)
    return fail(HIF8_ERR_INVALID_ARGUMENT,
                "%s: max_seq_len exceeds the block table capacity", name);
  if (max_seq_len > 0x7FFFFFFFll || batch > 0x7FFFFFFFll || num_heads > 0xFFFF)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: dimensions too large", name);
  if (batch == 0) return HIF8_OK;
  if (!query || !key_cache || !value_cache || !block_table || !seq_lens || !out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: null pointer argument", name);
  if (!aligned(key_cache, 4) || !aligned(value_cache, 4))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: caches must be 4-byte aligned", name);
  if (!aligned(query, 2) || !aligned(out, 2))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: query/out must be 2-byte aligned", name);

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
  p.log2_block_size = log2_of(block_size);
  p.hkv = int(num_kv_heads);
  p.hq = int(num_heads);
  p.group = int(num_heads / num_kv_heads);
  p.d = int(head_size);
  p.dv = int(head_size_v);
  p.max_len = int(max_seq_len);
  p.batch = int(batch);
  p.scale_log2 = scale * 1.4426950408889634f;
  const bool mfma = mfma_path(head_size, head_size_v, p.group, block_size, max_seq_len, query, out);
  if (mfma) {
    const SplitPlan plan = plan_splits(batch, num_kv_heads, max_seq_len);
    p.split_tokens = plan.split_tokens;
    p.num_splits = plan.num_splits;
    if (plan.num_splits > 1) {
      const size_t need = hif8_paged_decode_attention_workspace_size(batch, num_heads, num_kv_heads, head_size,
                                                                     head_size_v, max_seq_len);
      if (!workspace || workspace_bytes < need)
        return fail(HIF8_ERR_INVALID_ARGUMENT,
                    "%s: workspace of %zu bytes required (got %zu)", name, need,
                    workspace_bytes);
      if (!aligned(workspace, 16))
        return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: workspace must be 16-byte aligned", name);
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
  return check_launch(name);
}

}  // namespace
}  // namespace hif8

extern "C" int hif8_paged_decode_attention(const void *query, int q_dtype, const uint8_t *key_cache,
                                           const uint8_t *value_cache, int64_t num_blocks, int64_t block_size,
                                           int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
                                           const void *block_table, int block_table_dtype,
                                           int64_t max_blocks_per_seq, const int32_t *seq_lens, int64_t batch,
                                           int64_t num_heads, int64_t max_seq_len, float scale, void *out,
                                           void *workspace, size_t workspace_bytes, hif8_stream_t stream) {
  clear_error();
  return decode_attention("hif8_paged_decode_attention", query, q_dtype, key_cache, value_cache, num_blocks,
                          block_size, num_kv_heads, head_size, head_size_v, block_table, block_table_dtype,
                          max_blocks_per_seq, seq_lens, batch, num_heads, max_seq_len, scale, out, workspace,
                          workspace_bytes, stream);
}

// ------------------------------------------------- allocation-free variant

namespace hif8 {
namespace {

// The split partials of hif8_paged_decode_attention_noalloc: one array per
// GPU, held until the process ends.  Host code never uses `scratch` itself
// (on the host it names a stand-in, not device memory): it resolves each
// device's address once with hipGetSymbolAddress and passes that.
constexpr size_t kScratchBytes = size_t(HIF8_DECODE_ATTENTION_SCRATCH_BYTES);
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxScratchDevices = 64;

// This device's address of `scratch`, resolved on the first call per device
// (with that device current) and kept.
int scratch_address(const char *name, void **out) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxScratchDevices)
    return fail(HIF8_ERR_LAUNCH, "%s: no usable current HIP device", name);
  static std::mutex lock;
  static void *address[kMaxScratchDevices] = {};
  std::lock_guard<std::mutex> guard(lock);
  if (!address[device]) {
    void *ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return fail(HIF8_ERR_LAUNCH, "%s: cannot resolve the scratch array on device %d: %s", name, device,
                  hipGetErrorString(err));
    address[device] = ptr;
  }
  *out = address[device];
  return HIF8_OK;
}

}  // namespace
}  // namespace hif8

extern "C" int hif8_paged_decode_attention_noalloc(const void *query, int q_dtype, const uint8_t *key_cache,
                                                   const uint8_t *value_cache, int64_t num_blocks,
                                                   int64_t block_size, int64_t num_kv_heads, int64_t head_size,
                                                   int64_t head_size_v, const void *block_table,
                                                   int block_table_dtype, int64_t max_blocks_per_seq,
                                                   const int32_t *seq_lens, int64_t batch, int64_t num_heads,
                                                   int64_t max_seq_len, float scale, void *out,
                                                   hif8_stream_t stream) {
  static const char *kName = "hif8_paged_decode_attention_noalloc";
  clear_error();
  // The same split plan (hence the same results) as hif8_paged_decode_attention;
  // the partials go to this device's scratch array, which bounds the sizes.
  const size_t need = batch > 0 && max_seq_len > 0
                          ? hif8_paged_decode_attention_workspace_size(batch, num_heads, num_kv_heads, head_size,
                                                                       head_size_v, max_seq_len)
                          : 0;
  if (need > kScratchBytes)
    return fail(HIF8_ERR_UNSUPPORTED,
                "%s: these sizes need %zu bytes of split partials, more than the %zu-byte scratch array; "
                "call hif8_paged_decode_attention with a workspace instead",
                kName, need, kScratchBytes);
  void *ws = nullptr;
  if (need > 0) {
    if (const int st = scratch_address(kName, &ws)) return st;
  }
  return decode_attention(kName, query, q_dtype, key_cache, value_cache, num_blocks, block_size, num_kv_heads,
                          head_size, head_size_v, block_table, block_table_dtype, max_blocks_per_seq, seq_lens,
                          batch, num_heads, max_seq_len, scale, out, ws, need > 0 ? kScratchBytes : 0, stream);
}
