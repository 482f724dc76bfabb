// HiF8 token-embedding gather-decode for gfx950.
//
// Contract (AscendW8A8HiFloat8SoftLinearMethod.embedding, scheme.py:121-131):
//   rows   = weight[ids]                 (uint8 [T, D])
//   scales = weight_scale[ids]           (float32 [T])
//   out    = bf16(decode_bf16(rows) * bf16(scales))
// i.e. the codes go through the bf16 decode table, the row scale is rounded to
// bf16 first, and the product (exact in FP32: two 8-bit significands) is
// rounded once to bf16, as torch multiplies two bf16 tensors.
//
// One thread handles 16 consecutive codes of one token row (one 16-byte load,
// two 16-byte stores); ids outside [0, vocab) produce zero rows and are
// counted in *invalid (if given) so a caller can raise without a host sync.
#include "hif8_common.h"

namespace hif8 {
namespace {

constexpr int kThreads = 256;

template <typename IdT, bool kVec>
__global__ __launch_bounds__(kThreads) void embedding_kernel(const IdT *__restrict__ ids, int64_t tokens,
                                                             const uint8_t *__restrict__ table,
                                                             const float *__restrict__ table_scale,
                                                             int64_t vocab, int64_t dim,
                                                             uint16_t *__restrict__ out,
                                                             int32_t *__restrict__ invalid) {
  __shared__ float lut[256];
  lut[threadIdx.x] = __uint_as_float(kDeviceTables.decode_f32[threadIdx.x]);
  __syncthreads();
  const int64_t per_row = kVec ? dim / 16 : dim;
  const int64_t total = tokens * per_row;
  const int64_t step = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < total; i += step) {
    const int64_t t = i / per_row;
    const int64_t col = (i - t * per_row) * (kVec ? 16 : 1);
    const int64_t id = int64_t(ids[t]);
    uint16_t *dst = out + t * dim + col;
    const bool ok = id >= 0 && id < vocab;
    if (!ok) {
      if (invalid && col == 0) atomicAdd(invalid, 1);
      if constexpr (kVec) {
        reinterpret_cast<uint4 *>(dst)[0] = make_uint4(0, 0, 0, 0);
        reinterpret_cast<uint4 *>(dst)[1] = make_uint4(0, 0, 0, 0);
      } else {
        *dst = 0;
      }
      continue;
    }
    // bf16(scale), back to FP32 (exact).
    const float s = __uint_as_float(uint32_t(float_to_bf16_bits(table_scale[id])) << 16);
    const uint8_t *src = table + id * dim + col;
    if constexpr (kVec) {
      const uint4 q = *reinterpret_cast<const uint4 *>(src);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
      uint32_t o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t word = w[j >> 1] >> ((j & 1) * 16);
        const uint32_t h0 = float_to_bf16_bits(lut[word & 0xFFu] * s);
        const uint32_t h1 = float_to_bf16_bits(lut[(word >> 8) & 0xFFu] * s);
        o[j] = h0 | (h1 << 16);
      }
      uint4 *d = reinterpret_cast<uint4 *>(dst);
      d[0] = make_uint4(o[0], o[1], o[2], o[3]);
      d[1] = make_uint4(o[4], o[5], o[6], o[7]);
    } else {
      *dst = float_to_bf16_bits(lut[*src] * s);
    }
  }
}

template <typename IdT>
void launch(const IdT *ids, int64_t tokens, const uint8_t *table, const float *scale, int64_t vocab,
            int64_t dim, uint16_t *out, int32_t *invalid, hipStream_t stream, bool vec) {
  const int64_t items = tokens * (vec ? dim / 16 : dim);
  int64_t blocks = (items + kThreads - 1) / kThreads;
  if (blocks > 256 * 8) blocks = 256 * 8;
  if (blocks < 1) blocks = 1;
  if (vec)
    embedding_kernel<IdT, true><<<unsigned(blocks), kThreads, 0, stream>>>(ids, tokens, table, scale, vocab, dim,
                                                                          out, invalid);
  else
    embedding_kernel<IdT, false><<<unsigned(blocks), kThreads, 0, stream>>>(ids, tokens, table, scale, vocab, dim,
                                                                           out, invalid);
}

}  // namespace
}  // namespace hif8

using namespace hif8;

extern "C" int hif8_embedding_lookup(const void *ids, int ids_dtype, int64_t tokens, const uint8_t *table,
                                     const float *table_scale, int64_t vocab, int64_t dim, uint16_t *out,
                                     int32_t *invalid_ids, hif8_stream_t stream) {
  clear_error();
  if (!ids || !table || !table_scale || !out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_embedding_lookup: null pointer argument");
  if (tokens <= 0 || vocab <= 0 || dim <= 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_embedding_lookup: dimensions must be positive");
  if (ids_dtype != HIF8_INDEX_INT32 && ids_dtype != HIF8_INDEX_INT64)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_embedding_lookup: ids must be int32 or int64");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = dim % 16 == 0 && aligned(table, 16) && aligned(out, 16);
  if (ids_dtype == HIF8_INDEX_INT32)
    launch(static_cast<const int32_t *>(ids), tokens, table, table_scale, vocab, dim, out, invalid_ids, s, vec);
  else
    launch(static_cast<const int64_t *>(ids), tokens, table, table_scale, vocab, dim, out, invalid_ids, s, vec);
  return check_launch("hif8_embedding_lookup");
}
