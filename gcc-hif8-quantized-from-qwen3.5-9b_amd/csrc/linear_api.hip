// C-ABI entry points of the soft HiF8 linear operators: validation mirrors
// ValidateSoftLinear / SoftHif8StaticFusedGemm (hif8_native.cpp:241-316,784-861),
// then M <= 4 goes to the GEMV kernel and larger M to the MFMA GEMM.
#include "linear.h"

using namespace hif8;

namespace {

int validate(const char *op, const void *act, const uint8_t *weight, const float *act_scale,
             const float *channel_scale, const void *bias, int bias_dtype, const void *out,
             int out_dtype, int64_t m, int64_t n, int64_t k) {
  if (!act || !weight || !act_scale || !channel_scale || !out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: null pointer argument", op);
  if (m <= 0 || n <= 0 || k <= 0)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: dimensions must be positive, got M=%lld N=%lld K=%lld",
                op, (long long)m, (long long)n, (long long)k);
  if (m > 0x7FFFFFFFll || n > 0x7FFFFFFFll || k > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: dimensions must fit int32", op);
  if (!is_io_dtype(out_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "output_dtype must be torch.float16 or torch.bfloat16");
  if (bias && !is_io_dtype(bias_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "bias must have dtype torch.float16 or torch.bfloat16");
  if (!bias && bias_dtype != HIF8_DTYPE_NONE && !is_io_dtype(bias_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: invalid bias dtype code %d", op, bias_dtype);
  return HIF8_OK;
}

LinearArgs codes_args(const uint8_t *activation, const uint8_t *weight, const float *token_scale,
                      const float *channel_scale, const void *bias, int bias_dtype, void *out,
                      int out_dtype, int64_t m, int64_t n, int64_t k, hif8_stream_t stream) {
  LinearArgs a;
  a.act = activation;
  a.act_kind = kActCodes;
  a.act_scale = token_scale;
  a.weight = weight;
  a.channel_scale = channel_scale;
  a.bias = bias;
  a.bias_dtype = bias ? bias_dtype : HIF8_DTYPE_NONE;
  a.out = out;
  a.out_dtype = out_dtype;
  a.m = m;
  a.n = n;
  a.k = k;
  a.stream = reinterpret_cast<hipStream_t>(stream);
  return a;
}

}  // namespace

extern "C" int soft_hif8_gemv(const uint8_t *activation, const uint8_t *weight,
                              const float *token_scale, const float *channel_scale,
                              const void *bias, int bias_dtype, void *out, int out_dtype,
                              int64_t m, int64_t n, int64_t k, hif8_stream_t stream) {
  clear_error();
  int st = validate("soft_hif8_gemv", activation, weight, token_scale, channel_scale, bias,
                    bias_dtype, out, out_dtype, m, n, k);
  if (st) return st;
  if (m > 2) return fail(HIF8_ERR_INVALID_ARGUMENT, "soft_hif8_gemv requires M <= 2");
  return launch_gemv(codes_args(activation, weight, token_scale, channel_scale, bias, bias_dtype,
                                out, out_dtype, m, n, k, stream));
}

extern "C" int hif8_gate_up_silu_mul_quant(const uint8_t *activation, const uint8_t *weight,
                                           const float *token_scale, const float *channel_scale,
                                           const float *input_scale, uint8_t *codes, float *row_scale, int64_t m,
                                           int64_t inter, int64_t k, hif8_stream_t stream) {
  clear_error();
  int st = validate("hif8_gate_up_silu_mul_quant", activation, weight, token_scale, channel_scale, nullptr,
                    HIF8_DTYPE_NONE, codes, HIF8_DTYPE_BF16, m, 2 * inter, k);
  if (st) return st;
  if (!input_scale || !row_scale) return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gate_up_silu_mul_quant: null pointer argument");
  if (m > 4 || inter > 0x3FFFFFFFll)
    return fail(HIF8_ERR_UNSUPPORTED, "hif8_gate_up_silu_mul_quant takes 1 <= M <= 4 and inter < 2^30");
  LinearArgs a = codes_args(activation, weight, token_scale, channel_scale, nullptr, HIF8_DTYPE_NONE, nullptr,
                            HIF8_DTYPE_BF16, m, 2 * inter, k, stream);
  a.pair.inter = int(inter);
  a.pair.qs = input_scale;
  a.pair.codes = codes;
  a.pair.row_scale = row_scale;
  return launch_gemv(a);
}

extern "C" int hif8_linear_conv(const uint8_t *activation, const uint8_t *weight, const float *token_scale,
                                const float *channel_scale, uint16_t *out, const uint16_t *conv_weight,
                                uint16_t *conv_state, float *conv_out, int64_t m, int64_t n, int64_t k,
                                int64_t channels, int64_t conv_width, hif8_stream_t stream) {
  clear_error();
  int st = validate("hif8_linear_conv", activation, weight, token_scale, channel_scale, nullptr, HIF8_DTYPE_NONE,
                    out, HIF8_DTYPE_BF16, m, n, k);
  if (st) return st;
  if (!conv_weight || !conv_state || !conv_out)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_linear_conv: null pointer argument");
  if (channels <= 0 || channels > n || conv_width < 2 || conv_width > 4 || m * channels > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_linear_conv: needs 0 < channels <= n and 2 <= conv_width <= 4");
  LinearArgs a = codes_args(activation, weight, token_scale, channel_scale, nullptr, HIF8_DTYPE_NONE, out,
                            HIF8_DTYPE_BF16, m, n, k, stream);
  GemvConv conv;
  conv.channels = int(channels);
  conv.kw = int(conv_width);
  conv.weight = conv_weight;
  conv.state = conv_state;
  conv.out = conv_out;
  if (m <= 4) {
    a.conv = conv;
    st = launch_gemv(a);
    if (st != HIF8_ERR_UNSUPPORTED) return st;
    // The plan has no conv epilogue: the projection, then the conv on its own.
    clear_error();
    a.conv = GemvConv();
    st = launch_gemv(a);
  } else {
    st = launch_gemm(a);
  }
  if (st) return st;
  return launch_conv_rows(conv, out, n, m, reinterpret_cast<hipStream_t>(stream));
}

extern "C" size_t soft_hif8_gemm_workspace_size(int64_t m, int64_t n, int64_t k) {
  return gemm_workspace_size(m, n, k);
}

extern "C" int soft_hif8_gemm_with_workspace(const uint8_t *activation, const uint8_t *weight,
                                             const float *token_scale, const float *channel_scale,
                                             const void *bias, int bias_dtype, void *out,
                                             int out_dtype, int64_t m, int64_t n, int64_t k,
                                             void *workspace, size_t workspace_bytes,
                                             hif8_stream_t stream) {
  clear_error();
  int st = validate("soft_hif8_gemm", activation, weight, token_scale, channel_scale, bias,
                    bias_dtype, out, out_dtype, m, n, k);
  if (st) return st;
  const size_t need = gemm_workspace_size(m, n, k);
  if (workspace && workspace_bytes < need)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "soft_hif8_gemm: workspace of %zu bytes, %zu required",
                workspace_bytes, need);
  if (workspace && !aligned(workspace, 256))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "soft_hif8_gemm: workspace must be 256-byte aligned");
  LinearArgs a = codes_args(activation, weight, token_scale, channel_scale, bias, bias_dtype, out,
                            out_dtype, m, n, k, stream);
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return m <= 4 ? launch_gemv(a) : launch_gemm(a);
}

extern "C" int soft_hif8_gemm(const uint8_t *activation, const uint8_t *weight,
                              const float *token_scale, const float *channel_scale,
                              const void *bias, int bias_dtype, void *out, int out_dtype,
                              int64_t m, int64_t n, int64_t k, hif8_stream_t stream) {
  return soft_hif8_gemm_with_workspace(activation, weight, token_scale, channel_scale, bias,
                                       bias_dtype, out, out_dtype, m, n, k, nullptr, 0, stream);
}

extern "C" int hif8_decode_bf16(const uint8_t *codes, uint16_t *out, int64_t elements, hif8_stream_t stream) {
  clear_error();
  if (!codes || !out) return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_decode_bf16: null pointer argument");
  if (elements < 0 || elements % 16)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_decode_bf16: element count must be a non-negative multiple of 16, got %lld",
                (long long)elements);
  if (!aligned(codes, 16) || !aligned(out, 16))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_decode_bf16: buffers must be 16-byte aligned");
  if (elements == 0) return HIF8_OK;
  return launch_decode_bf16(codes, out, size_t(elements), reinterpret_cast<hipStream_t>(stream));
}

extern "C" size_t soft_hif8_gemm_decoded_weight_workspace_size(int64_t m, int64_t n, int64_t k) {
  return gemm_decoded_weight_workspace_size(m, n, k);
}

extern "C" int soft_hif8_gemm_decoded_weight(const uint8_t *activation, const uint16_t *weight_bf16,
                                             const float *token_scale, const float *channel_scale,
                                             const void *bias, int bias_dtype, void *out, int out_dtype,
                                             int64_t m, int64_t n, int64_t k, void *workspace,
                                             size_t workspace_bytes, hif8_stream_t stream) {
  clear_error();
  const char *op = "soft_hif8_gemm_decoded_weight";
  int st = validate(op, activation, reinterpret_cast<const uint8_t *>(weight_bf16), token_scale, channel_scale,
                    bias, bias_dtype, out, out_dtype, m, n, k);
  if (st) return st;
  if (k % 64) return fail(HIF8_ERR_UNSUPPORTED, "%s: K must be a multiple of 64, got %lld", op, (long long)k);
  if (!aligned(activation, 16) || !aligned(weight_bf16, 16))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: activation and weight must be 16-byte aligned", op);
  const size_t need = gemm_decoded_weight_workspace_size(m, n, k);
  if (!workspace || workspace_bytes < need)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: workspace of %zu bytes, %zu required", op, workspace_bytes, need);
  if (!aligned(workspace, 256)) return fail(HIF8_ERR_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned", op);
  LinearArgs a = codes_args(activation, nullptr, token_scale, channel_scale, bias, bias_dtype, out, out_dtype, m,
                            n, k, stream);
  a.weight_bf16 = weight_bf16;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return launch_gemm_decoded_weight(a);
}

extern "C" int soft_hif8_static_fused_gemm(const void *x, int x_dtype, const uint8_t *weight,
                                           const float *fixed_scale, const float *channel_scale,
                                           const void *bias, int bias_dtype, void *out,
                                           int out_dtype, int64_t m, int64_t n, int64_t k,
                                           hif8_stream_t stream) {
  clear_error();
  int st = validate("soft_hif8_static_fused_gemm", x, weight, fixed_scale, channel_scale, bias,
                    bias_dtype, out, out_dtype, m, n, k);
  if (st) return st;
  if (!is_io_dtype(x_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "activation must have dtype torch.float16 or torch.bfloat16");
  if (m > 4) return fail(HIF8_ERR_INVALID_ARGUMENT, "soft_hif8_static_fused_gemm requires M <= 4");
  LinearArgs a = codes_args(nullptr, weight, fixed_scale, channel_scale, bias, bias_dtype, out,
                            out_dtype, m, n, k, stream);
  a.act = x;
  a.act_kind = x_dtype == HIF8_DTYPE_BF16 ? kActBf16 : kActF16;
  return launch_gemv(a);
}

extern "C" int soft_hif8_fused_gemm(const void *x, int x_dtype, const uint8_t *weight,
                                    const float *channel_scale, const void *bias, int bias_dtype, void *out,
                                    int out_dtype, int64_t m, int64_t n, int64_t k, hif8_stream_t stream) {
  clear_error();
  // No activation-scale argument: every row's scale is its own finite amax.
  int st = validate("soft_hif8_fused_gemm", x, weight, channel_scale, channel_scale, bias, bias_dtype, out,
                    out_dtype, m, n, k);
  if (st) return st;
  if (!is_io_dtype(x_dtype))
    return fail(HIF8_ERR_INVALID_ARGUMENT, "activation must have dtype torch.float16 or torch.bfloat16");
  if (m > 2) return fail(HIF8_ERR_INVALID_ARGUMENT, "soft_hif8_fused_gemm requires M <= 2");
  LinearArgs a = codes_args(nullptr, weight, nullptr, channel_scale, bias, bias_dtype, out, out_dtype, m, n, k,
                            stream);
  a.act = x;
  a.act_kind = x_dtype == HIF8_DTYPE_BF16 ? kActBf16Dyn : kActF16Dyn;
  return launch_gemv(a);
}

extern "C" int hif8_gemv_launch_plan(int64_t m, int64_t n, int64_t k, int activation_kind, char *kernel,
                                     size_t kernel_len, int64_t *grid) {
  clear_error();
  if (m < 1 || m > 4 || n <= 0 || k <= 0 || n > 0x7FFFFFFFll || k > 0x7FFFFFFFll)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gemv_launch_plan: needs 1 <= M <= 4 and positive N, K");
  if (activation_kind < HIF8_ACT_CODES || activation_kind > HIF8_ACT_BF16_STATIC)
    return fail(HIF8_ERR_INVALID_ARGUMENT, "hif8_gemv_launch_plan: unknown activation kind %d", activation_kind);
  static_assert(HIF8_ACT_CODES == kActCodes && HIF8_ACT_F16_STATIC == kActF16 && HIF8_ACT_BF16_STATIC == kActBf16,
                "activation kind codes");
  return describe_gemv(m, n, k, activation_kind, kernel, kernel_len, grid);
}
