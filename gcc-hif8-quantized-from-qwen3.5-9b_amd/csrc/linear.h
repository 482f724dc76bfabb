// Internal launch interface shared by the GEMV, GEMM and C-ABI units.
#pragma once

#include "hif8_common.h"

namespace hif8 {

enum ActKind : int {
  kActCodes = 0,  // uint8 HiF8 activation codes + token_scale[m]
  kActF16 = 1,    // float16 x, statically quantised in the kernel with fixed_scale[0]
  kActBf16 = 2,   // bfloat16 x, likewise
  kActF16Dyn = 3,   // float16 x, quantised in the kernel with its per-row dynamic scale
  kActBf16Dyn = 4,  // bfloat16 x, likewise
};

// The gate_up projection of an MLP fused with SiLU-mul and the down
// projection's static input quant (inter > 0): weight rows [0, inter) are the
// gates, [inter, 2 inter) the ups; a GEMV block takes kR / 2 gate rows and the
// matching up rows, and writes codes[m, i] = static HiF8 code of
// bf16(silu(bf16 gate) * bf16 up) with the fixed scale qs[0] (the arithmetic of
// hif8_silu_mul_quant over the bf16 GEMV output) and row_scale[m] = qs[0].
struct GemvPair {
  int inter = 0;
  const float *qs = nullptr;
  uint8_t *codes = nullptr;
  float *row_scale = nullptr;
};

// Causal depthwise-conv epilogue of a decode token's qkvz projection: for
// output rows c < channels of activation row m, with x = the bf16 output
// value, out[m, c] = SiLU(sum_t bf(state[m, c, t]) bf(weight[c, t]) +
// x bf(weight[c, kw - 1])) in fp32 (t = 0 .. kw - 2 in order), and
// state[m, c] shifts by one with x appended.  2 <= kw <= 4, bf16 output.
struct GemvConv {
  int channels = 0;
  int kw = 0;
  const uint16_t *weight = nullptr;  // [channels, kw] bf16
  uint16_t *state = nullptr;         // [m, channels, kw - 1] bf16
  float *out = nullptr;              // [m, channels]
};

struct LinearArgs {
  const void *act;        // [m, k] codes or fp16/bf16 x
  int act_kind;           // ActKind
  const float *act_scale; // token_scale[m] (codes) or fixed_scale[1] (x)
  const uint8_t *weight;  // [n, k]
  const float *channel_scale;  // [n]
  const void *bias;       // [n] or nullptr
  int bias_dtype;         // HIF8_DTYPE_*
  void *out;              // [m, n]
  int out_dtype;          // HIF8_DTYPE_FP16 / HIF8_DTYPE_BF16
  int64_t m, n, k;
  hipStream_t stream;
  void *workspace = nullptr;    // split-K partials (GEMM only), may be null
  size_t workspace_bytes = 0;
  const uint16_t *weight_bf16 = nullptr;  // [n, k] weight decoded beforehand (GEMM), else null
  GemvPair pair;                          // GEMV only: gate_up + SiLU-mul + quant epilogue
  GemvConv conv;                          // GEMV only: causal-conv epilogue
};

// HBM-streaming GEMV for m <= 4 (gemv.hip).  Returns a status; with a.pair
// set, HIF8_ERR_UNSUPPORTED where the plan is not the dot2 kernel; with
// a.conv set, HIF8_ERR_UNSUPPORTED where it is neither the dot2 nor the
// MFMA-4 kernel.
int launch_gemv(const LinearArgs &a);
// The conv epilogue of a.conv as a kernel of its own over y [m, ld] bf16 (the
// projection output), for plans without the epilogue.
int launch_conv_rows(const GemvConv &conv, const uint16_t *y, int64_t ld, int64_t m, hipStream_t stream);
// The kernel launch_gemv picks for these sizes and activation kind (16-byte
// aligned operands): its name as profilers print it, and its grid.
int describe_gemv(int64_t m, int64_t n, int64_t k, int act_kind, char *name, size_t name_len, int64_t *grid);
// bf16-MFMA GEMM for any m (gemm.hip).  Returns a status.  With a workspace of
// gemm_workspace_size(m, n, k) bytes, shapes with too few output tiles to fill
// the chip split K over several blocks; without one they run unsplit.
int launch_gemm(const LinearArgs &a);
size_t gemm_workspace_size(int64_t m, int64_t n, int64_t k);
// The GEMM with the weight already decoded to bf16 (a.weight_bf16; a.weight is
// not read): the activation codes are decoded into the workspace and both
// operands stream into LDS by DMA.  Needs k % 64 == 0, 16-byte aligned
// operands and a 256-byte aligned workspace of
// gemm_decoded_weight_workspace_size(m, n, k) bytes (checked by the caller).
int launch_gemm_decoded_weight(const LinearArgs &a);
size_t gemm_decoded_weight_workspace_size(int64_t m, int64_t n, int64_t k);
// HiF8 codes -> bf16 (elements % 16 == 0, 16-byte aligned buffers).
int launch_decode_bf16(const uint8_t *codes, uint16_t *out, size_t elements, hipStream_t stream);

}  // namespace hif8
