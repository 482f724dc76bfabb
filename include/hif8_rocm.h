/*
 * hif8_rocm.h - C ABI of the MI355X (gfx950) HiFloat8 static W8A8KV8 hot path.
 *
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream, enqueues its kernels on that stream and returns without a host
 * synchronisation.  Nothing here allocates device memory.  The return value is
 * HIF8_OK or an error code; hif8_last_error() returns the message of the last
 * failure on the calling thread.  Arguments are validated before any launch, so
 * a failed call has not touched device memory.
 *
 * Each function cites the reference interface it replaces (paths relative to
 * the reference repository root).  The reference reaches its Ascend kernels
 * through ACLNN's two-phase GetWorkspaceSize + execute calls from a torch-npu
 * bridge; here the same operators are one call each, and the single operator
 * that needs scratch memory (paged decode attention) reports its size through
 * a separate query so the caller owns that memory.
 *
 * Layout conventions (all row-major, contiguous):
 *   HiF8 byte tensors          uint8
 *   scales                     float32
 *   activations / bias / out   fp16 or bf16, selected by HIF8_DTYPE_*
 */
#ifndef HIF8_ROCM_H
#define HIF8_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A hipStream_t; NULL selects the legacy default stream. */
typedef void *hif8_stream_t;

enum hif8_status {
  HIF8_OK = 0,
  HIF8_ERR_INVALID_ARGUMENT = 1, /* shape/dtype/pointer contract violated */
  HIF8_ERR_UNSUPPORTED = 2,      /* valid request outside what the kernels implement */
  HIF8_ERR_LAUNCH = 3            /* the HIP runtime rejected a launch */
};

/* Numeric codes match the reference bridge (hif8_native.cpp:32-33). */
enum hif8_dtype {
  HIF8_DTYPE_FP16 = 0,
  HIF8_DTYPE_BF16 = 1,
  HIF8_DTYPE_NONE = -1 /* "no bias" */
};

/* Integer index tensors (slot mappings, block tables). */
enum hif8_index_dtype {
  HIF8_INDEX_INT32 = 0,
  HIF8_INDEX_INT64 = 1
};

/* Message of the last failed call on this thread ("" if none). */
const char *hif8_last_error(void);

/* Version of this ABI (bumped on any signature change). */
int hif8_abi_version(void);

/*
 * Static activation quantisation.
 * Replaces aclnnHif8StaticQuant as called by Hif8StaticQuant
 * (csrc/extension/hif8_native.cpp:487-554; kernel csrc/opp/op_kernel/hif8_static_quant.cpp:37-150).
 *   x          [rows, k] fp16/bf16
 *   fixed_scale[scale_count] float32, finite > 0; row r uses fixed_scale[r % scale_count]
 *   data       [rows, k] uint8  <- enc_sat(float(x) / scale)   (IEEE division)
 *   row_scale  [rows] float32   <- fixed_scale[r % scale_count] (contiguous; the
 *              reference returns a stride-16 view of the same values)
 */
int hif8_static_quant(const void *x, int x_dtype, int64_t rows, int64_t k,
                      const float *fixed_scale, int64_t scale_count,
                      uint8_t *data, float *row_scale, hif8_stream_t stream);

/*
 * Dynamic per-row activation quantisation (the legacy W8A8HIF8_SOFT scheme).
 * Replaces aclnnHif8DynamicQuant as called by Hif8DynamicQuant
 * (csrc/extension/hif8_native.cpp:433-485; kernel csrc/opp/op_kernel/hif8_dynamic_quant.cpp:35-200).
 *   x         [rows, k] fp16/bf16
 *   row_scale [rows] float32 <- max(max |x[r, :]| over finite values, 1e-12)
 *             (contiguous; the reference returns a stride-16 view)
 *   data      [rows, k] uint8 <- enc(float(x) * RN(1 / row_scale)) when k % 32 == 0,
 *             enc(float(x) / row_scale) otherwise (the reference's vector and
 *             scalar paths); NaN -> 0x80, Inf kept, zero magnitude unsigned
 */
int hif8_dynamic_quant(const void *x, int x_dtype, int64_t rows, int64_t k, uint8_t *data,
                       float *row_scale, hif8_stream_t stream);

/*
 * Scaled decode to bf16.
 * Replaces aclnnHif8ScaledDecode as called by Hif8ScaledDecode
 * (csrc/extension/hif8_native.cpp:556-611; kernel csrc/opp/op_kernel/hif8_scaled_decode.cpp:50-125).
 *   data  [rows, k] uint8 with row pitch data_row_stride bytes (>= k; lets the
 *         caller decode KV rows in place, skipping the inline 4-byte scale)
 *   scale [rows] float32
 *   out   [rows, k] bf16 payloads <- bf16_RNE(dec(b) * scale[r]); NaN -> 0x7FC0
 */
int hif8_scaled_decode(const uint8_t *data, int64_t rows, int64_t k, int64_t data_row_stride,
                       const float *scale, uint16_t *out, hif8_stream_t stream);

/*
 * HiF8 token-embedding gather-decode.
 * Replaces AscendW8A8HiFloat8SoftLinearMethod.embedding
 * (src/vllm_ascend_hif8/scheme.py:121-131: index_select of weight rows and
 * weight_scale, bf16 decode table, product with bf16(scale)).
 *   ids [tokens] int32/int64 (ids_dtype HIF8_INDEX_*), table [vocab, dim] uint8,
 *   table_scale [vocab] float32, out [tokens, dim] bf16:
 *     out[t] = bf16(decode_bf16(table[ids[t]]) * bf16(table_scale[ids[t]]))
 *   ids outside [0, vocab) give zero rows and, if invalid_ids is not NULL, add
 *   one each to *invalid_ids (the caller raises, as index_select would).
 */
int hif8_embedding_lookup(const void *ids, int ids_dtype, int64_t tokens, const uint8_t *table,
                          const float *table_scale, int64_t vocab, int64_t dim, uint16_t *out,
                          int32_t *invalid_ids, hif8_stream_t stream);

/*
 * Soft-decode GEMV, reference contract M <= 2.
 * Replaces aclnnSoftHif8Gemv as called by SoftHif8Gemv
 * (csrc/extension/hif8_native.cpp:241-316,613-631; kernel csrc/opp/op_kernel/soft_hif8_gemv.cpp:28-317).
 *   activation [m, k] uint8, weight [n, k] uint8,
 *   token_scale [m], channel_scale [n] float32,
 *   bias [n] fp16/bf16 or NULL (bias_dtype HIF8_DTYPE_NONE),
 *   out [m, n] fp16/bf16:
 *     out = RNE((sum_k dec(a) dec(w)) * token_scale[m] * channel_scale[n] + bias[n])
 *   with FP32 accumulation.
 */
int soft_hif8_gemv(const uint8_t *activation, const uint8_t *weight, const float *token_scale,
                   const float *channel_scale, const void *bias, int bias_dtype, void *out,
                   int out_dtype, int64_t m, int64_t n, int64_t k, hif8_stream_t stream);

/*
 * Soft-decode GEMM, any M >= 1 (same arguments and contract as soft_hif8_gemv).
 * Replaces aclnnSoftHif8Gemm / aclnnSoftHif8PrefillGemm as routed by SoftHif8Gemm
 * (csrc/extension/hif8_native.cpp:633-669; kernel csrc/opp/op_kernel/soft_hif8_gemm.cpp:163-2139).
 * M <= 4 runs the HBM-streaming GEMV kernel, larger M the bf16-MFMA kernel.
 */
int soft_hif8_gemm(const uint8_t *activation, const uint8_t *weight, const float *token_scale,
                   const float *channel_scale, const void *bias, int bias_dtype, void *out,
                   int out_dtype, int64_t m, int64_t n, int64_t k, hif8_stream_t stream);

/*
 * Bytes of workspace soft_hif8_gemm_with_workspace uses for these sizes (0: none).
 * First phase of the reference's two-phase call, aclnnSoftHif8GemmGetWorkspaceSize
 * (csrc/extension/hif8_native.cpp:386-425).
 */
size_t soft_hif8_gemm_workspace_size(int64_t m, int64_t n, int64_t k);

/*
 * soft_hif8_gemm with a caller-owned workspace: the second phase,
 * aclnnSoftHif8Gemm(workspace, size, executor, stream) (hif8_native.cpp:228-239,386-425).
 * With workspace_bytes >= soft_hif8_gemm_workspace_size(m, n, k) (256-byte aligned)
 * the activation codes are decoded once into the workspace (bf16) instead of once
 * per output column tile, and shapes with too few output tiles to fill the GPU
 * split K into FP32 partials added in a fixed order (deterministic).  With NULL
 * the call equals soft_hif8_gemm (same results up to FP32 summation order).  A
 * non-NULL workspace that is too small or misaligned is an error.
 */
int soft_hif8_gemm_with_workspace(const uint8_t *activation, const uint8_t *weight,
                                  const float *token_scale, const float *channel_scale,
                                  const void *bias, int bias_dtype, void *out, int out_dtype,
                                  int64_t m, int64_t n, int64_t k, void *workspace,
                                  size_t workspace_bytes, hif8_stream_t stream);

/*
 * Prefill GEMM over a weight kept decoded to bf16.  No counterpart in the
 * reference (its GEMM reads the uint8 weight every call): for callers that
 * trade memory for speed (2 bytes per weight element, 18 GB for a 9B model,
 * on 288 GB of HBM) and keep hif8_decode_bf16(weight) next to the codes.
 * Same arguments and results as soft_hif8_gemm_with_workspace (within FP32
 * summation order) for any M >= 1, with weight_bf16 [n, k] in place of the
 * codes; requires K % 64 == 0, 16-byte aligned activation and weight, and a
 * 256-byte aligned workspace of soft_hif8_gemm_decoded_weight_workspace_size
 * bytes (the decoded activation and split-K partials).
 */
size_t soft_hif8_gemm_decoded_weight_workspace_size(int64_t m, int64_t n, int64_t k);
int soft_hif8_gemm_decoded_weight(const uint8_t *activation, const uint16_t *weight_bf16,
                                  const float *token_scale, const float *channel_scale,
                                  const void *bias, int bias_dtype, void *out, int out_dtype,
                                  int64_t m, int64_t n, int64_t k, void *workspace,
                                  size_t workspace_bytes, hif8_stream_t stream);

/*
 * Plain decode of HiF8 codes to bf16 payloads (exact: every HiF8 value is a
 * bf16 value; NaN 0x80 -> 0x7FC0), elements % 16 == 0, 16-byte aligned
 * buffers.  No counterpart in the reference; builds the weight that
 * soft_hif8_gemm_decoded_weight reads.
 */
int hif8_decode_bf16(const uint8_t *codes, uint16_t *out, int64_t elements, hif8_stream_t stream);

/*
 * Fixed-scale fused quant + GEMM for M <= 4.
 * Replaces aclnnSoftHif8StaticFusedGemm as called by SoftHif8StaticFusedGemm
 * (csrc/extension/hif8_native.cpp:784-910; kernel csrc/opp/op_kernel/soft_hif8_fused_gemm.cpp
 * built with HIF8_FUSED_STATIC_SCALE=1).  Equal, bit for bit, to hif8_static_quant
 * followed by soft_hif8_gemm with token_scale = fixed_scale[0].
 *   x [m, k] fp16/bf16 (x_dtype), fixed_scale [1] float32, other arguments as above.
 */
int soft_hif8_static_fused_gemm(const void *x, int x_dtype, const uint8_t *weight,
                                const float *fixed_scale, const float *channel_scale,
                                const void *bias, int bias_dtype, void *out, int out_dtype,
                                int64_t m, int64_t n, int64_t k, hif8_stream_t stream);

/*
 * Dynamic-scale fused quant + GEMM for M <= 2 (the legacy soft scheme's
 * HIF8_SOFT_FUSED_GENERATION path).
 * Replaces aclnnSoftHif8FusedGemm as called by SoftHif8FusedGemm
 * (csrc/extension/hif8_native.cpp:671-782; kernel csrc/opp/op_kernel/soft_hif8_fused_gemm.cpp
 * with the dynamic scale, lines 445-571 and 720-745):
 *   s[m] = max(finite amax of x[m, :], 1e-12);  a = dec(enc(float(x) / s[m]))  (IEEE division)
 *   out[m, n] = sum_k a[m, k] dec(w[n, k]) * s[m] * channel_scale[n] (+ bias[n])
 *   x [m, k] fp16/bf16 (x_dtype); other arguments as soft_hif8_gemm.
 */
int soft_hif8_fused_gemm(const void *x, int x_dtype, const uint8_t *weight, const float *channel_scale,
                         const void *bias, int bias_dtype, void *out, int out_dtype, int64_t m, int64_t n,
                         int64_t k, hif8_stream_t stream);

/*
 * Introspection, no counterpart in the reference: the GEMV kernel that soft_hif8_gemm
 * (activation_kind HIF8_ACT_CODES) or soft_hif8_static_fused_gemm (HIF8_ACT_F16_STATIC /
 * HIF8_ACT_BF16_STATIC, M = 1; the op itself runs static quant + the code kernel at
 * M >= 2) launches for these sizes with 16-byte aligned operands: its name as profilers
 * print it (template arguments included) into kernel[kernel_len], and its grid in
 * workgroups.  For benchmarks that must match their timing to a profile of the same
 * kernel.  Returns HIF8_OK or an error status; launches nothing.
 */
#define HIF8_ACT_CODES 0
#define HIF8_ACT_F16_STATIC 1
#define HIF8_ACT_BF16_STATIC 2
int hif8_gemv_launch_plan(int64_t m, int64_t n, int64_t k, int activation_kind, char *kernel, size_t kernel_len,
                          int64_t *grid);

/*
 * Fused static KV-cache write (quantise + pack + scatter in one launch).
 * Replaces the static branch of _write_hif8_cache
 * (src/vllm_ascend_hif8/kv_runtime.py:1222-1339): _quantize_kv with checkpoint
 * per-head scales (kv_runtime.py:1168-1199, i.e. aclnnHif8StaticQuant on
 * [tokens * Hkv, D] rows with S = Hkv), pack_kv_rows (kv_cache.py:151-170) and
 * the slot index_copy_ (kv_runtime.py:1313-1316).
 *   key [tokens, Hkv, D], value [tokens, Hkv, Dv]   fp16/bf16 (x_dtype)
 *   key_scale, value_scale [Hkv] float32, finite > 0
 *   slot_mapping [tokens] int32/int64 (slot_dtype): flat slot block * block_size + offset;
 *                slot < 0 is a padding token and is skipped
 *   key_cache [num_blocks, block_size, Hkv, D + 4], value_cache [..., Dv + 4] uint8, in place:
 *     row = enc_sat(x / scale[h]) codes followed by scale[h] (4 bytes, little-endian)
 *   invalid_slots  optional int32 counter (may be NULL): incremented once per token whose
 *                  slot is >= num_blocks * block_size; such tokens are not written.  The
 *                  caller zeroes it.  (The reference raises IndexError after a host check.)
 * D and Dv must be divisible by 4 (kv_cache.py:48-57).
 */
int hif8_kv_cache_write(const void *key, const void *value, int x_dtype, int64_t tokens,
                        int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
                        const float *key_scale, const float *value_scale,
                        const void *slot_mapping, int slot_dtype,
                        uint8_t *key_cache, uint8_t *value_cache, int64_t num_blocks,
                        int64_t block_size, int32_t *invalid_slots, hif8_stream_t stream);

/*
 * Bytes of workspace hif8_paged_decode_attention needs for these sizes (0 if none).
 * The split plan depends only on these arguments.  Mirrors ACLNN's GetWorkspaceSize
 * phase (csrc/extension/hif8_native.cpp:202-239).
 */
size_t hif8_paged_decode_attention_workspace_size(int64_t batch, int64_t num_heads,
                                                  int64_t num_kv_heads, int64_t head_size,
                                                  int64_t head_size_v, int64_t max_seq_len);

/*
 * Paged HiF8 decode attention, one query token per request.
 * Replaces the decode branch of _forward_hif8_attention
 * (src/vllm_ascend_hif8/kv_runtime.py:1470-1563): gather_kv_rows_concat
 * (kv_cache.py:255-311) + scaled decode (kv_runtime.py:1201-1211) +
 * torch_npu.npu_fused_infer_attention_score (kv_runtime.py:1526-1540), whose
 * contract is paged_attention_reference (kv_cache.py:314-372).  Pages are
 * decoded inside the kernel; nothing is materialised.
 *   query [batch, num_heads, D] fp16/bf16 (q_dtype)
 *   key_cache / value_cache as written by hif8_kv_cache_write
 *   block_table [batch, max_blocks_per_seq] int32/int64
 *   seq_lens [batch] int32 on the device; each is clamped to [0, max_seq_len]
 *   max_seq_len <= max_blocks_per_seq * block_size, >= every seq_len
 *   out [batch, num_heads, Dv] in the query dtype:
 *     out[b, h] = softmax(scale * q[b, h] . K_b^T) V_b over the request's seq_lens[b]
 *     tokens with K/V rows dec(code) * row scale and KV head h / (num_heads / Hkv);
 *     a request with no tokens gets zeros; tokens whose block id lies outside
 *     [0, num_blocks) are left out (the caller validates the table).
 *   workspace  at least hif8_paged_decode_attention_workspace_size(...) bytes, 16-byte
 *              aligned (may be NULL when that size is 0)
 */
int hif8_paged_decode_attention(const void *query, int q_dtype, const uint8_t *key_cache,
                                const uint8_t *value_cache, int64_t num_blocks, int64_t block_size,
                                int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
                                const void *block_table, int block_table_dtype,
                                int64_t max_blocks_per_seq, const int32_t *seq_lens, int64_t batch,
                                int64_t num_heads, int64_t max_seq_len, float scale, void *out,
                                void *workspace, size_t workspace_bytes, hif8_stream_t stream);

/*
 * hif8_paged_decode_attention without a workspace argument, allocating nothing.
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels, split plan and results as
 * hif8_paged_decode_attention; the split partials live in a file-scope device
 * array of HIF8_DECODE_ATTENTION_SCRATCH_BYTES per GPU, held until the process
 * ends.  Sizes whose workspace (hif8_paged_decode_attention_workspace_size) exceeds
 * that array are rejected with HIF8_ERR_UNSUPPORTED before any launch (e.g. batch 4
 * at 16384 tokens needs 8.5 MB and fits; batch 64 at 16384 does not).  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (other streams,
 * other host threads) race and must be serialised by the caller.
 */
#define HIF8_DECODE_ATTENTION_SCRATCH_BYTES (16u << 20)
int hif8_paged_decode_attention_noalloc(const void *query, int q_dtype, const uint8_t *key_cache,
                                        const uint8_t *value_cache, int64_t num_blocks, int64_t block_size,
                                        int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
                                        const void *block_table, int block_table_dtype,
                                        int64_t max_blocks_per_seq, const int32_t *seq_lens, int64_t batch,
                                        int64_t num_heads, int64_t max_seq_len, float scale, void *out,
                                        hif8_stream_t stream);

/*
 * Bytes of workspace hif8_paged_prefill_attention needs for these sizes (0 if none);
 * the plan (image slots, key splits) depends only on these arguments (ACLNN
 * GetWorkspaceSize phase, csrc/extension/hif8_native.cpp:202-239).  Requests whose
 * query covers more than two 64-row tiles (rows = tokens x query heads per KV head)
 * get decoded tile images while the images of all such requests fit 512 MiB; the
 * others decode their pages inside the attention kernel.
 */
size_t hif8_paged_prefill_attention_workspace_size(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                                                   int64_t head_size, int64_t head_size_v,
                                                   int64_t total_query_tokens, int64_t max_query_len,
                                                   int64_t max_seq_len);

/*
 * Paged HiF8 attention for several query tokens per request: prefill and chunked
 * prefill.  Replaces the TND branch of _forward_hif8_attention
 * (src/vllm_ascend_hif8/kv_runtime.py:1470-1563, the sequence plan of
 * _attention_sequence_plan :588-641, npu_fused_infer_attention_score with
 * sparse_mode=3 when causal) whose contract is paged_attention_reference with
 * query_lens (kv_cache.py:314-372).  Pages are decoded inside the kernel.
 *   query [total_query_tokens, num_heads, D] fp16/bf16 (TND layout)
 *   query_start_loc [batch + 1] int32 on the device: request b owns query rows
 *     query_start_loc[b] .. query_start_loc[b + 1] - 1 (the reference's cumulative
 *     actual_seq_lengths_q is query_start_loc[1:]); rows from query_start_loc[batch]
 *     to total_query_tokens - 1 are not written
 *   seq_lens [batch] int32 on the device: cached tokens of each request after this
 *     step's cache write, clamped to [0, max_seq_len]
 *   max_query_len >= every request's query length (sizes the grid)
 *   causal: query row i of request b sits at position seq_lens[b] - q_len_b + i and
 *     sees keys 0 .. that position (right-aligned mask, kv_cache.py:365-369); 0: every
 *     row sees all seq_lens[b] keys
 *   out [total_query_tokens, num_heads, Dv] in the query dtype, K/V rows decoded to the
 *     query dtype as dtype(dec(code) * row scale) (kv_cache.py:355-356); a row that sees
 *     no key gets zeros; tokens whose block id lies outside [0, num_blocks) are left out
 *   workspace  at least hif8_paged_prefill_attention_workspace_size(...) bytes, 16-byte
 *              aligned (may be NULL when that size is 0)
 */
int hif8_paged_prefill_attention(const void *query, int q_dtype, const uint8_t *key_cache,
                                 const uint8_t *value_cache, int64_t num_blocks, int64_t block_size,
                                 int64_t num_kv_heads, int64_t head_size, int64_t head_size_v,
                                 const void *block_table, int block_table_dtype, int64_t max_blocks_per_seq,
                                 const int32_t *query_start_loc, const int32_t *seq_lens, int64_t batch,
                                 int64_t num_heads, int64_t total_query_tokens, int64_t max_query_len,
                                 int64_t max_seq_len, float scale, int causal, void *out, void *workspace,
                                 size_t workspace_bytes, hif8_stream_t stream);

/*
 * Decode-step glue of the synthetic hybrid model (the end-to-end workload).
 * These have no counterpart among the reference's operators: they fuse the
 * bf16 / fp32 model parts that the reference leaves to vLLM (norms, the MLP
 * activation, the linear-attention conv and recurrence), so that a decode
 * step is a few launches per layer.  All tensors bf16 unless stated.
 *
 * hif8_add_rms_norm: per row of h [rows, n]: if delta is not NULL,
 *   h <- bf16(h + delta) in place; out = bf16(h * rsqrt(mean(h^2) + eps) * weight).
 * hif8_silu_mul: gate_up [rows, 2n] -> out [rows, n] = bf16(silu(gate) * up).
 * hif8_qk_norm_rope: one decode token of full attention: qkv [batch, (Hq + 2 Hkv) D] ->
 *   q_out [batch, Hq, D], k_out / v_out [batch, Hkv, D]; q and k heads RMS-normalised
 *   (q_norm / k_norm [D]) then rotated on the first rotary_dim dims (halves i, i + r/2,
 *   angle pos[b] * inv_freq[i], float32 inv_freq [r/2], int64 pos [batch]); if slots is
 *   not NULL, slots[b] = block_table[b, pos / block_size] * block_size + pos % block_size
 *   (int32 block_table [batch, max_blocks]), or -1 (a padding slot the cache write
 *   skips) when pos < 0, pos / block_size >= max_blocks or the table entry is negative.
 *   D <= 256.
 * hif8_gdn_decode_step: one token of the gated delta rule for batch requests.
 *   mixed_qkvz [batch, ld]: q | k (k_heads x k_dim each) | v | z (v_heads x v_dim each)
 *   ba [batch, 2 v_heads]: b | a;  conv_weight [C, conv_width], C = 2 k_heads k_dim + v_heads v_dim;
 *   conv_state [batch, C, conv_width - 1] (updated); a_log, dt_bias [v_heads] float32;
 *   rec_state [batch, v_heads, k_dim, v_dim] float32 (updated); out_norm [v_dim];
 *   out [batch, v_heads * v_dim]; conv_scratch [batch, C] float32 workspace.
 *   k_dim, v_dim <= 128; v_heads a multiple of k_heads.
 */
/* out [m, n] = bf16(x [m, k] weight [n, k]^T), FP32 accumulation, 1 <= m <= 4,
 * k % 8 == 0, 16-byte aligned bf16 operands: the decode step's small bf16
 * projections (glue, no reference counterpart). */
int hif8_bf16_gemv(const uint16_t *x, const uint16_t *weight, uint16_t *out, int64_t m, int64_t n, int64_t k,
                   hif8_stream_t stream);
int hif8_add_rms_norm(uint16_t *h, const uint16_t *delta, const uint16_t *weight, uint16_t *out,
                      int64_t rows, int64_t n, float eps, hif8_stream_t stream);
int hif8_silu_mul(const uint16_t *gate_up, uint16_t *out, int64_t rows, int64_t n, hif8_stream_t stream);
/* The two above with the next projection's static input quant fused in (glue,
 * no reference counterpart): also codes [rows, n] = the hif8_static_quant
 * codes of their bf16 result with the fixed scale input_scale[0] (float32
 * [1]) and row_scale [rows] = input_scale[0], so that the projection runs
 * straight from codes.  hif8_add_rms_norm_quant still writes out; both need
 * n % 8 == 0 (the norm also n <= 8192), 16-byte aligned bf16 rows and
 * 8-byte aligned codes, else HIF8_ERR_UNSUPPORTED. */
int hif8_add_rms_norm_quant(uint16_t *h, const uint16_t *delta, const uint16_t *weight, uint16_t *out,
                            const float *input_scale, uint8_t *codes, float *row_scale, int64_t rows, int64_t n,
                            float eps, hif8_stream_t stream);
int hif8_silu_mul_quant(const uint16_t *gate_up, const float *input_scale, uint8_t *codes, float *row_scale,
                        int64_t rows, int64_t n, hif8_stream_t stream);
/* The gate_up projection and hif8_silu_mul_quant in one GEMV launch (glue, no
 * reference counterpart): weight [2 inter, k] (gate rows, then up rows) and
 * channel_scale [2 inter] as for soft_hif8_gemm over activation codes [m, k]
 * with token_scale [m]; codes [m, inter] and row_scale [m] equal
 * hif8_silu_mul_quant(soft_hif8_gemm(...) in bf16, input_scale) bit for bit.
 * 1 <= m <= 4; HIF8_ERR_UNSUPPORTED where the GEMV plan for (m, 2 inter, k)
 * is not the dot2 kernel (then run the two calls). */
int hif8_gate_up_silu_mul_quant(const uint8_t *activation, const uint8_t *weight, const float *token_scale,
                                const float *channel_scale, const float *input_scale, uint8_t *codes,
                                float *row_scale, int64_t m, int64_t inter, int64_t k, hif8_stream_t stream);
/* The qkvz projection of a linear-attention decode token with the causal
 * depthwise conv in its epilogue (glue, no reference counterpart): out [m, n]
 * = soft_hif8_gemm(activation codes, weight, token_scale, channel_scale) in
 * bf16, and for the first `channels` columns (q | k | v) conv_out [m,
 * channels] (float32) = SiLU(sum_t bf(conv_state[m, c, t]) bf(conv_weight[c,
 * t]) + out[m, c] bf(conv_weight[c, kw - 1])) (t = 0 .. kw - 2 in order), the
 * conv of hif8_gdn_decode_step, with conv_state [m, channels, kw - 1] shifted
 * by one and out[m, c] appended.  2 <= conv_width <= 4.  One launch where the
 * GEMV plan for (m, n, k) is the dot2 or MFMA-4 kernel, else the projection
 * and a conv kernel. */
int hif8_linear_conv(const uint8_t *activation, const uint8_t *weight, const float *token_scale,
                     const float *channel_scale, uint16_t *out, const uint16_t *conv_weight, uint16_t *conv_state,
                     float *conv_out, int64_t m, int64_t n, int64_t k, int64_t channels, int64_t conv_width,
                     hif8_stream_t stream);
/* The recurrence of hif8_gdn_decode_token from the conv outputs of
 * hif8_linear_conv (glue, no reference counterpart): conv [batch, channels]
 * float32, mixed_qkvz [batch, ld] (the z gate columns after the channels),
 * the b/a projection of x [batch, hidden] by ba_weight [2 v_heads, hidden]
 * folded in; one block per (request, value head).  Outputs and states equal
 * hif8_gdn_decode_token's given the same conv outputs.  Needs k_dim in
 * {32, 64, 128}, v_dim <= 128, hidden % 8 == 0, hidden <= 8192 and 16-byte
 * aligned x and ba_weight, else HIF8_ERR_UNSUPPORTED. */
int hif8_gdn_decode_head(const float *conv, const uint16_t *mixed_qkvz, int64_t ld, const uint16_t *x,
                         const uint16_t *ba_weight, int64_t hidden, const float *a_log, const float *dt_bias,
                         float *rec_state, const uint16_t *out_norm, uint16_t *out, int64_t batch, int64_t k_heads,
                         int64_t v_heads, int64_t k_dim, int64_t v_dim, float eps, hif8_stream_t stream);
int hif8_qk_norm_rope(const uint16_t *qkv, const uint16_t *q_norm, const uint16_t *k_norm, const int64_t *pos,
                      const float *inv_freq, const int32_t *block_table, int64_t max_blocks, int64_t block_size,
                      uint16_t *q_out, uint16_t *k_out, uint16_t *v_out, int64_t *slots, int64_t batch,
                      int64_t num_heads, int64_t num_kv_heads, int64_t head_size, int64_t rotary_dim, float eps,
                      hif8_stream_t stream);
int hif8_gdn_decode_step(const uint16_t *mixed_qkvz, int64_t ld, const uint16_t *ba,
                         const uint16_t *conv_weight, uint16_t *conv_state, const float *a_log,
                         const float *dt_bias, float *rec_state, const uint16_t *out_norm, uint16_t *out,
                         float *conv_scratch, int64_t batch, int64_t k_heads, int64_t v_heads, int64_t k_dim,
                         int64_t v_dim, int64_t conv_width, float eps, hif8_stream_t stream);
/* hif8_gdn_decode_step with the b/a projection folded in (glue, no reference
 * counterpart): ba = hif8_bf16_gemv(x [batch, hidden], ba_weight [2 v_heads,
 * hidden]) computed inside, one launch instead of three; the conv state equals
 * the two calls' bit for bit, b and a equal hif8_bf16_gemv's, the recurrent
 * state and output agree to FP32 rounding (the state dot products are scaled
 * by the q / k norms after the sum).  Needs v_heads / k_heads <= 2,
 * k_dim % 8 == 0, k_dim, v_dim <= 128, hidden % 8 == 0, hidden <= 8192,
 * conv_width <= 4 and 16-byte aligned x and ba_weight, else
 * HIF8_ERR_UNSUPPORTED (run the two calls). */
int hif8_gdn_decode_token(const uint16_t *mixed_qkvz, int64_t ld, const uint16_t *x, const uint16_t *ba_weight,
                          int64_t hidden, const uint16_t *conv_weight, uint16_t *conv_state, const float *a_log,
                          const float *dt_bias, float *rec_state, const uint16_t *out_norm, uint16_t *out,
                          int64_t batch, int64_t k_heads, int64_t v_heads, int64_t k_dim, int64_t v_dim,
                          int64_t conv_width, float eps, hif8_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HIF8_ROCM_H */
