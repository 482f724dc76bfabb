// Thin torch extension over the C ABI in include/hif8_rocm.h.
//
// Registers the reference's operator schemas under the same namespace
// (pybind.cpp:6-13) so callers of torch.ops.vllm_ascend_hif8.* switch over
// unchanged, with implementations for HIP tensors (torch's "cuda" key on ROCm)
// and Meta implementations for shape inference (pybind.cpp:27-89).  Each
// implementation validates like the reference bridge (hif8_native.cpp:131-316,
// 487-611, 784-861), allocates outputs with the caching allocator and calls
// the C ABI on the current HIP stream.  No host synchronisation, no fallback.
// Two operators are new: the fused KV-cache write and the paged decode
// attention that replace the reference's quant + pack + index_copy_ and
// gather + decode + fused-attention sequences (kv_runtime.py:1222-1563).
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include "hif8_rocm.h"

namespace {

void CheckDeviceTensor(const at::Tensor &t, const char *name) {
  TORCH_CHECK(t.defined(), name, " must be defined");
  TORCH_CHECK(t.is_cuda(), name, " must be a HIP device tensor, got ", t.device());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.storage_offset() == 0, name, " must have storage_offset == 0");
}

void CheckSameDevice(const at::Tensor &t, const at::Device &d, const char *name) {
  TORCH_CHECK(t.device() == d, name, " must be on ", d, ", got ", t.device());
}

void CheckPositiveDimensions(const at::Tensor &t, const char *name) {
  for (int64_t i = 0; i < t.dim(); ++i)
    TORCH_CHECK(t.size(i) > 0, name, " dimensions must be positive, got ", t.sizes());
}

void CheckFitsUint32(int64_t v, const char *name) {
  TORCH_CHECK(v > 0 && v <= int64_t(0xFFFFFFFFll), name, " must fit a positive uint32, got ", v);
}

int DtypeCode(at::ScalarType t) {
  return t == at::ScalarType::BFloat16 ? HIF8_DTYPE_BF16 : HIF8_DTYPE_FP16;
}

hif8_stream_t CurrentStream(const at::Device &d) {
  return reinterpret_cast<hif8_stream_t>(c10::hip::getCurrentHIPStream(d.index()).stream());
}

void CheckStatus(int status, const char *op) {
  TORCH_CHECK(status == HIF8_OK, op, " failed: ", hif8_last_error());
}

void ValidateSoftLinear(const at::Tensor &activation, const at::Tensor &weight,
                        const at::Tensor &token_scale, const at::Tensor &channel_scale,
                        const c10::optional<at::Tensor> &bias, at::ScalarType output_dtype,
                        bool gemv, at::ScalarType weight_dtype = at::ScalarType::Byte) {
  CheckDeviceTensor(activation, "activation");
  CheckDeviceTensor(weight, "weight");
  CheckDeviceTensor(token_scale, "token_scale");
  CheckDeviceTensor(channel_scale, "channel_scale");
  TORCH_CHECK(activation.scalar_type() == at::ScalarType::Byte, "activation must have dtype torch.uint8");
  TORCH_CHECK(weight.scalar_type() == weight_dtype, weight_dtype == at::ScalarType::Byte
                                                       ? "weight must have dtype torch.uint8"
                                                       : "weight must have dtype torch.bfloat16 (decoded HiF8)");
  TORCH_CHECK(token_scale.scalar_type() == at::ScalarType::Float, "token_scale must have dtype torch.float32");
  TORCH_CHECK(channel_scale.scalar_type() == at::ScalarType::Float, "channel_scale must have dtype torch.float32");
  TORCH_CHECK(activation.dim() == 2, "activation must have shape [M, K]");
  TORCH_CHECK(weight.dim() == 2, "weight must have shape [N, K]");
  TORCH_CHECK(token_scale.dim() == 1, "token_scale must have shape [M]");
  TORCH_CHECK(channel_scale.dim() == 1, "channel_scale must have shape [N]");
  CheckPositiveDimensions(activation, "activation");
  CheckPositiveDimensions(weight, "weight");
  const int64_t m = activation.size(0), k = activation.size(1), n = weight.size(0);
  TORCH_CHECK(weight.size(1) == k, "activation and weight K dimensions differ: ", k, " != ", weight.size(1));
  TORCH_CHECK(token_scale.numel() == m, "token_scale must contain one value per activation row");
  TORCH_CHECK(channel_scale.numel() == n, "channel_scale must contain one value per output channel");
  TORCH_CHECK(gemv ? m <= 2 : m > 0, gemv ? "soft_hif8_gemv requires M <= 2" : "soft_hif8_gemm requires M > 0");
  CheckFitsUint32(m, "M");
  CheckFitsUint32(n, "N");
  CheckFitsUint32(k, "K");
  const auto device = activation.device();
  CheckSameDevice(weight, device, "weight");
  CheckSameDevice(token_scale, device, "token_scale");
  CheckSameDevice(channel_scale, device, "channel_scale");
  if (bias.has_value()) {
    CheckDeviceTensor(*bias, "bias");
    CheckSameDevice(*bias, device, "bias");
    TORCH_CHECK(bias->dim() == 1, "bias must have shape [N]");
    TORCH_CHECK(bias->numel() == n, "bias must contain N values");
    TORCH_CHECK(bias->scalar_type() == at::ScalarType::Half || bias->scalar_type() == at::ScalarType::BFloat16,
                "bias must have dtype torch.float16 or torch.bfloat16");
  }
  TORCH_CHECK(output_dtype == at::ScalarType::Half || output_dtype == at::ScalarType::BFloat16,
              "output_dtype must be torch.float16 or torch.bfloat16");
}

using LinearFn = int (*)(const uint8_t *, const uint8_t *, const float *, const float *, const void *, int,
                         void *, int, int64_t, int64_t, int64_t, hif8_stream_t);

at::Tensor SoftLinear(const at::Tensor &activation, const at::Tensor &weight, const at::Tensor &token_scale,
                      const at::Tensor &channel_scale, const c10::optional<at::Tensor> &bias,
                      at::ScalarType output_dtype, bool gemv, const char *op, LinearFn fn) {
  ValidateSoftLinear(activation, weight, token_scale, channel_scale, bias, output_dtype, gemv);
  const c10::OptionalDeviceGuard guard(activation.device());
  auto out = at::empty({activation.size(0), weight.size(0)}, activation.options().dtype(output_dtype));
  const void *bias_ptr = bias.has_value() ? bias->data_ptr() : nullptr;
  const int bias_dtype = bias.has_value() ? DtypeCode(bias->scalar_type()) : HIF8_DTYPE_NONE;
  CheckStatus(fn(activation.data_ptr<uint8_t>(), weight.data_ptr<uint8_t>(), token_scale.data_ptr<float>(),
                 channel_scale.data_ptr<float>(), bias_ptr, bias_dtype, out.data_ptr(), DtypeCode(output_dtype),
                 activation.size(0), weight.size(0), activation.size(1), CurrentStream(activation.device())),
              op);
  return out;
}

std::tuple<at::Tensor, at::Tensor> Hif8StaticQuant(const at::Tensor &x, const at::Tensor &fixed_scale) {
  CheckDeviceTensor(x, "x");
  CheckDeviceTensor(fixed_scale, "fixed_scale");
  TORCH_CHECK(x.scalar_type() == at::ScalarType::Half || x.scalar_type() == at::ScalarType::BFloat16,
              "x must have dtype torch.float16 or torch.bfloat16");
  TORCH_CHECK(fixed_scale.scalar_type() == at::ScalarType::Float, "fixed_scale must have dtype torch.float32");
  TORCH_CHECK(x.dim() >= 1, "x must have at least one dimension");
  TORCH_CHECK(fixed_scale.dim() == 1, "fixed_scale must have shape [scale_count]");
  CheckPositiveDimensions(x, "x");
  CheckPositiveDimensions(fixed_scale, "fixed_scale");
  const int64_t k = x.size(-1);
  const int64_t rows = x.numel() / k;
  TORCH_CHECK(rows % fixed_scale.numel() == 0, "fixed_scale count must divide the activation row count");
  CheckFitsUint32(rows, "activation row count");
  CheckFitsUint32(k, "K");
  CheckFitsUint32(fixed_scale.numel(), "fixed scale count");
  CheckSameDevice(fixed_scale, x.device(), "fixed_scale");
  const c10::OptionalDeviceGuard guard(x.device());
  auto data = at::empty(x.sizes(), x.options().dtype(at::ScalarType::Byte));
  auto row_scale = at::empty({rows}, x.options().dtype(at::ScalarType::Float));
  CheckStatus(hif8_static_quant(x.data_ptr(), DtypeCode(x.scalar_type()), rows, k, fixed_scale.data_ptr<float>(),
                                fixed_scale.numel(), data.data_ptr<uint8_t>(), row_scale.data_ptr<float>(),
                                CurrentStream(x.device())),
              "hif8_static_quant");
  return {data, row_scale};
}

// hif8_native.cpp:433-485 (Hif8DynamicQuant): row scales are returned
// contiguous [rows] rather than as a stride-16 view.
std::tuple<at::Tensor, at::Tensor> Hif8DynamicQuant(const at::Tensor &x) {
  CheckDeviceTensor(x, "x");
  TORCH_CHECK(x.scalar_type() == at::ScalarType::Half || x.scalar_type() == at::ScalarType::BFloat16,
              "x must have dtype torch.float16 or torch.bfloat16");
  TORCH_CHECK(x.dim() >= 1, "x must have at least one dimension");
  CheckPositiveDimensions(x, "x");
  const int64_t k = x.size(-1);
  const int64_t rows = x.numel() / k;
  CheckFitsUint32(rows, "activation row count");
  CheckFitsUint32(k, "K");
  const c10::OptionalDeviceGuard guard(x.device());
  auto data = at::empty(x.sizes(), x.options().dtype(at::ScalarType::Byte));
  auto row_scale = at::empty({rows}, x.options().dtype(at::ScalarType::Float));
  CheckStatus(hif8_dynamic_quant(x.data_ptr(), DtypeCode(x.scalar_type()), rows, k, data.data_ptr<uint8_t>(),
                                 row_scale.data_ptr<float>(), CurrentStream(x.device())),
              "hif8_dynamic_quant");
  return {data, row_scale};
}

at::Tensor Hif8ScaledDecode(const at::Tensor &data, const at::Tensor &scale) {
  CheckDeviceTensor(data, "data");
  CheckDeviceTensor(scale, "scale");
  TORCH_CHECK(data.scalar_type() == at::ScalarType::Byte, "data must have dtype torch.uint8");
  TORCH_CHECK(scale.scalar_type() == at::ScalarType::Float, "scale must have dtype torch.float32");
  TORCH_CHECK(data.dim() == 2, "data must have shape [rows, K]");
  TORCH_CHECK(scale.dim() == 1, "scale must have shape [rows]");
  CheckPositiveDimensions(data, "data");
  TORCH_CHECK(scale.numel() == data.size(0), "scale must contain one value per data row");
  CheckFitsUint32(data.size(0), "row count");
  CheckFitsUint32(data.size(1), "K");
  CheckSameDevice(scale, data.device(), "scale");
  const c10::OptionalDeviceGuard guard(data.device());
  auto out = at::empty(data.sizes(), data.options().dtype(at::ScalarType::BFloat16));
  CheckStatus(hif8_scaled_decode(data.data_ptr<uint8_t>(), data.size(0), data.size(1), data.size(1),
                                 scale.data_ptr<float>(), reinterpret_cast<uint16_t *>(out.data_ptr()),
                                 CurrentStream(data.device())),
              "hif8_scaled_decode");
  return out;
}

at::Tensor SoftHif8Gemv(const at::Tensor &activation, const at::Tensor &weight, const at::Tensor &token_scale,
                        const at::Tensor &channel_scale, const c10::optional<at::Tensor> &bias,
                        at::ScalarType output_dtype) {
  return SoftLinear(activation, weight, token_scale, channel_scale, bias, output_dtype, true, "soft_hif8_gemv",
                    &soft_hif8_gemv);
}

at::Tensor SoftHif8Gemm(const at::Tensor &activation, const at::Tensor &weight, const at::Tensor &token_scale,
                        const at::Tensor &channel_scale, const c10::optional<at::Tensor> &bias,
                        at::ScalarType output_dtype) {
  ValidateSoftLinear(activation, weight, token_scale, channel_scale, bias, output_dtype, false);
  const c10::OptionalDeviceGuard guard(activation.device());
  const int64_t m = activation.size(0), n = weight.size(0), k = activation.size(1);
  auto out = at::empty({m, n}, activation.options().dtype(output_dtype));
  // Split-K workspace from the stream-ordered caching allocator, as the
  // reference takes its ACLNN workspace (hif8_native.cpp:202-226).
  const size_t ws_bytes = soft_hif8_gemm_workspace_size(m, n, k);
  at::Tensor ws;
  if (ws_bytes) ws = at::empty({int64_t(ws_bytes)}, activation.options().dtype(at::ScalarType::Byte));
  const void *bias_ptr = bias.has_value() ? bias->data_ptr() : nullptr;
  const int bias_dtype = bias.has_value() ? DtypeCode(bias->scalar_type()) : HIF8_DTYPE_NONE;
  CheckStatus(soft_hif8_gemm_with_workspace(
                  activation.data_ptr<uint8_t>(), weight.data_ptr<uint8_t>(), token_scale.data_ptr<float>(),
                  channel_scale.data_ptr<float>(), bias_ptr, bias_dtype, out.data_ptr(), DtypeCode(output_dtype),
                  m, n, k, ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, CurrentStream(activation.device())),
              "soft_hif8_gemm");
  return out;
}

// Prefill GEMM over a weight kept decoded to bf16 (no reference counterpart).
at::Tensor SoftHif8GemmDecodedWeight(const at::Tensor &activation, const at::Tensor &weight_bf16,
                                     const at::Tensor &token_scale, const at::Tensor &channel_scale,
                                     const c10::optional<at::Tensor> &bias, at::ScalarType output_dtype) {
  ValidateSoftLinear(activation, weight_bf16, token_scale, channel_scale, bias, output_dtype, false,
                     at::ScalarType::BFloat16);
  const c10::OptionalDeviceGuard guard(activation.device());
  const int64_t m = activation.size(0), n = weight_bf16.size(0), k = activation.size(1);
  TORCH_CHECK(k % 64 == 0, "soft_hif8_gemm_decoded_weight requires K % 64 == 0, got ", k);
  auto out = at::empty({m, n}, activation.options().dtype(output_dtype));
  const size_t ws_bytes = soft_hif8_gemm_decoded_weight_workspace_size(m, n, k);
  at::Tensor ws = at::empty({int64_t(ws_bytes)}, activation.options().dtype(at::ScalarType::Byte));
  const void *bias_ptr = bias.has_value() ? bias->data_ptr() : nullptr;
  const int bias_dtype = bias.has_value() ? DtypeCode(bias->scalar_type()) : HIF8_DTYPE_NONE;
  CheckStatus(soft_hif8_gemm_decoded_weight(
                  activation.data_ptr<uint8_t>(), reinterpret_cast<const uint16_t *>(weight_bf16.data_ptr()),
                  token_scale.data_ptr<float>(), channel_scale.data_ptr<float>(), bias_ptr, bias_dtype,
                  out.data_ptr(), DtypeCode(output_dtype), m, n, k, ws.data_ptr(), ws_bytes,
                  CurrentStream(activation.device())),
              "soft_hif8_gemm_decoded_weight");
  return out;
}

at::Tensor Hif8DecodeBf16(const at::Tensor &codes) {
  CheckDeviceTensor(codes, "codes");
  TORCH_CHECK(codes.scalar_type() == at::ScalarType::Byte, "codes must have dtype torch.uint8");
  TORCH_CHECK(codes.numel() % 16 == 0, "hif8_decode_bf16 requires a multiple of 16 elements, got ", codes.numel());
  const c10::OptionalDeviceGuard guard(codes.device());
  auto out = at::empty(codes.sizes(), codes.options().dtype(at::ScalarType::BFloat16));
  CheckStatus(hif8_decode_bf16(codes.data_ptr<uint8_t>(), reinterpret_cast<uint16_t *>(out.data_ptr()),
                               codes.numel(), CurrentStream(codes.device())),
              "hif8_decode_bf16");
  return out;
}

at::Tensor SoftHif8StaticFusedGemm(const at::Tensor &activation, const at::Tensor &weight,
                                   const at::Tensor &fixed_scale, const at::Tensor &channel_scale,
                                   const c10::optional<at::Tensor> &bias, at::ScalarType output_dtype) {
  CheckDeviceTensor(activation, "activation");
  CheckDeviceTensor(weight, "weight");
  CheckDeviceTensor(fixed_scale, "fixed_scale");
  CheckDeviceTensor(channel_scale, "channel_scale");
  TORCH_CHECK(activation.scalar_type() == at::ScalarType::Half || activation.scalar_type() == at::ScalarType::BFloat16,
              "activation must have dtype torch.float16 or torch.bfloat16");
  TORCH_CHECK(weight.scalar_type() == at::ScalarType::Byte, "weight must have dtype torch.uint8");
  TORCH_CHECK(fixed_scale.scalar_type() == at::ScalarType::Float, "fixed_scale must have dtype torch.float32");
  TORCH_CHECK(channel_scale.scalar_type() == at::ScalarType::Float, "channel_scale must have dtype torch.float32");
  TORCH_CHECK(activation.dim() == 2, "activation must have shape [M, K]");
  TORCH_CHECK(weight.dim() == 2, "weight must have shape [N, K]");
  TORCH_CHECK(fixed_scale.dim() == 1 && fixed_scale.numel() == 1, "fixed_scale must have shape [1]");
  TORCH_CHECK(channel_scale.dim() == 1, "channel_scale must have shape [N]");
  CheckPositiveDimensions(activation, "activation");
  CheckPositiveDimensions(weight, "weight");
  TORCH_CHECK(activation.size(0) <= 4, "soft_hif8_static_fused_gemm requires M <= 4");
  TORCH_CHECK(activation.size(1) == weight.size(1), "activation and weight K dimensions differ: ",
              activation.size(1), " != ", weight.size(1));
  TORCH_CHECK(channel_scale.numel() == weight.size(0), "channel_scale must contain one value per output channel");
  CheckFitsUint32(activation.size(0), "M");
  CheckFitsUint32(weight.size(0), "N");
  CheckFitsUint32(activation.size(1), "K");
  const auto device = activation.device();
  CheckSameDevice(weight, device, "weight");
  CheckSameDevice(fixed_scale, device, "fixed_scale");
  CheckSameDevice(channel_scale, device, "channel_scale");
  if (bias.has_value()) {
    CheckDeviceTensor(*bias, "bias");
    CheckSameDevice(*bias, device, "bias");
    TORCH_CHECK(bias->dim() == 1, "bias must have shape [N]");
    TORCH_CHECK(bias->numel() == weight.size(0), "bias must contain N values");
    TORCH_CHECK(bias->scalar_type() == at::ScalarType::Half || bias->scalar_type() == at::ScalarType::BFloat16,
                "bias must have dtype torch.float16 or torch.bfloat16");
  }
  TORCH_CHECK(output_dtype == at::ScalarType::Half || output_dtype == at::ScalarType::BFloat16,
              "output_dtype must be torch.float16 or torch.bfloat16");
  const c10::OptionalDeviceGuard guard(device);
  auto out = at::empty({activation.size(0), weight.size(0)}, activation.options().dtype(output_dtype));
  const void *bias_ptr = bias.has_value() ? bias->data_ptr() : nullptr;
  const int bias_dtype = bias.has_value() ? DtypeCode(bias->scalar_type()) : HIF8_DTYPE_NONE;
  const int64_t m = activation.size(0), n = weight.size(0), k = activation.size(1);
  // Widest N and K fused into one launch at M = 1 (tuning knobs
  // HIF8_FUSED_MAX_N / HIF8_FUSED_MAX_K, read once; no limit by default).
  static const int64_t max_n = [] {
    const char *v = getenv("HIF8_FUSED_MAX_N");
    return v && *v ? int64_t(atoll(v)) : INT64_MAX;
  }();
  static const int64_t max_k = [] {
    const char *v = getenv("HIF8_FUSED_MAX_K");
    return v && *v ? int64_t(atoll(v)) : INT64_MAX;
  }();
  // Several rows run as one launch where the fused kind's plan is the MFMA-4
  // GEMV (K <= 4096, M = 4, or M = 3 over N >= 16384) and N <= 2048 (tuning
  // knob HIF8_FUSED_MULTI_MAX_N, read once).  Every block re-encodes all M
  // rows (about 14 VALU operations per value), so the one launch wins only
  // where the grid is small; measured on MI355X in graphs at M = 4 against
  // static quant + GEMV: k/v 2048x4096 8.2 vs 8.5 us, q 4096x4096 11.5 vs
  // 10.2, gate_up 24576x4096 31.7 vs 23.9.
  static const int64_t multi_max_n = [] {
    const char *v = getenv("HIF8_FUSED_MULTI_MAX_N");
    return v && *v ? int64_t(atoll(v)) : int64_t(2048);
  }();
  bool multi_fused = false;
  if (m >= 2 && n <= multi_max_n) {
    char kernel[96] = {0};
    int64_t grid = 0;
    multi_fused = hif8_gemv_launch_plan(m, n, k, activation.scalar_type() == at::ScalarType::BFloat16
                                                     ? HIF8_ACT_BF16_STATIC : HIF8_ACT_F16_STATIC,
                                        kernel, sizeof(kernel), &grid) == HIF8_OK &&
                  strncmp(kernel, "gemv_mfma4_kernel", 17) == 0;
  }
  if (m >= 2 ? !multi_fused : (k > max_k || n > max_n)) {
    // Every block of the dot2 kernel's fused kinds encodes its whole
    // activation chunk, which costs more than a separate quant launch once
    // there are several rows (measured on MI355X in graphs at M = 4: q
    // 4096x4096 14.3 vs 9.9 us, gate_up 24576x4096 38.1 vs 26.6).  One row
    // is faster fused (q 6.5 vs 8.7-9.0 us, k/v 2048x4096 5.0-5.2 vs 7.6, o
    // 6.6-6.7 vs 8.3-8.8, 12288x4096 12.1-12.3 vs 13.7-14.0; since the
    // encode takes one slow-path branch per 16 values also gate_up
    // 24576x4096, 19.9-20.6 vs 21.2-21.7, and down 4096x12288 with its
    // chunk loop, 13.6-13.7 vs 14.1-14.2).
    // The two launches give the same codes and the same GEMV, hence equal
    // outputs.
    auto codes = at::empty({m, k}, activation.options().dtype(at::ScalarType::Byte));
    auto row_scale = at::empty({m}, activation.options().dtype(at::ScalarType::Float));
    const auto stream = CurrentStream(device);
    CheckStatus(hif8_static_quant(activation.data_ptr(), DtypeCode(activation.scalar_type()), m, k,
                                  fixed_scale.data_ptr<float>(), 1, codes.data_ptr<uint8_t>(),
                                  row_scale.data_ptr<float>(), stream),
                "soft_hif8_static_fused_gemm");
    CheckStatus(soft_hif8_gemm(codes.data_ptr<uint8_t>(), weight.data_ptr<uint8_t>(), row_scale.data_ptr<float>(),
                               channel_scale.data_ptr<float>(), bias_ptr, bias_dtype, out.data_ptr(),
                               DtypeCode(output_dtype), m, n, k, stream),
                "soft_hif8_static_fused_gemm");
    return out;
  }
  CheckStatus(soft_hif8_static_fused_gemm(activation.data_ptr(), DtypeCode(activation.scalar_type()),
                                          weight.data_ptr<uint8_t>(), fixed_scale.data_ptr<float>(),
                                          channel_scale.data_ptr<float>(), bias_ptr, bias_dtype, out.data_ptr(),
                                          DtypeCode(output_dtype), activation.size(0), weight.size(0),
                                          activation.size(1), CurrentStream(device)),
              "soft_hif8_static_fused_gemm");
  return out;
}

// hif8_native.cpp:671-782 (SoftHif8FusedGemm): dynamic per-row scale, M <= 2.
at::Tensor SoftHif8FusedGemm(const at::Tensor &activation, const at::Tensor &weight,
                             const at::Tensor &channel_scale, const c10::optional<at::Tensor> &bias,
                             at::ScalarType output_dtype) {
  CheckDeviceTensor(activation, "activation");
  CheckDeviceTensor(weight, "weight");
  CheckDeviceTensor(channel_scale, "channel_scale");
  TORCH_CHECK(activation.scalar_type() == at::ScalarType::Half || activation.scalar_type() == at::ScalarType::BFloat16,
              "activation must have dtype torch.float16 or torch.bfloat16");
  TORCH_CHECK(weight.scalar_type() == at::ScalarType::Byte, "weight must have dtype torch.uint8");
  TORCH_CHECK(channel_scale.scalar_type() == at::ScalarType::Float, "channel_scale must have dtype torch.float32");
  TORCH_CHECK(activation.dim() == 2, "activation must have shape [M, K]");
  TORCH_CHECK(weight.dim() == 2, "weight must have shape [N, K]");
  TORCH_CHECK(channel_scale.dim() == 1, "channel_scale must have shape [N]");
  CheckPositiveDimensions(activation, "activation");
  CheckPositiveDimensions(weight, "weight");
  TORCH_CHECK(activation.size(0) <= 2, "soft_hif8_fused_gemm requires M <= 2");
  TORCH_CHECK(activation.size(1) == weight.size(1), "activation and weight K dimensions differ: ",
              activation.size(1), " != ", weight.size(1));
  TORCH_CHECK(channel_scale.numel() == weight.size(0), "channel_scale must contain one value per output channel");
  CheckFitsUint32(activation.size(0), "M");
  CheckFitsUint32(weight.size(0), "N");
  CheckFitsUint32(activation.size(1), "K");
  const auto device = activation.device();
  CheckSameDevice(weight, device, "weight");
  CheckSameDevice(channel_scale, device, "channel_scale");
  if (bias.has_value()) {
    CheckDeviceTensor(*bias, "bias");
    CheckSameDevice(*bias, device, "bias");
    TORCH_CHECK(bias->dim() == 1, "bias must have shape [N]");
    TORCH_CHECK(bias->numel() == weight.size(0), "bias must contain N values");
    TORCH_CHECK(bias->scalar_type() == at::ScalarType::Half || bias->scalar_type() == at::ScalarType::BFloat16,
                "bias must have dtype torch.float16 or torch.bfloat16");
  }
  TORCH_CHECK(output_dtype == at::ScalarType::Half || output_dtype == at::ScalarType::BFloat16,
              "output_dtype must be torch.float16 or torch.bfloat16");
  const c10::OptionalDeviceGuard guard(device);
  auto out = at::empty({activation.size(0), weight.size(0)}, activation.options().dtype(output_dtype));
  const void *bias_ptr = bias.has_value() ? bias->data_ptr() : nullptr;
  const int bias_dtype = bias.has_value() ? DtypeCode(bias->scalar_type()) : HIF8_DTYPE_NONE;
  CheckStatus(soft_hif8_fused_gemm(activation.data_ptr(), DtypeCode(activation.scalar_type()),
                                   weight.data_ptr<uint8_t>(), channel_scale.data_ptr<float>(), bias_ptr, bias_dtype,
                                   out.data_ptr(), DtypeCode(output_dtype), activation.size(0), weight.size(0),
                                   activation.size(1), CurrentStream(device)),
              "soft_hif8_fused_gemm");
  return out;
}


// ---------------------------------------------------------------- KV cache
// The KV operators take views as they come (the cache of a layer is usually a
// view into one large allocation), so they need contiguity, not offset 0.

void CheckContiguousDevice(const at::Tensor &t, const char *name) {
  TORCH_CHECK(t.defined(), name, " must be defined");
  TORCH_CHECK(t.is_cuda(), name, " must be a HIP device tensor, got ", t.device());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

int IndexCode(const at::Tensor &t, const char *name) {
  TORCH_CHECK(t.scalar_type() == at::ScalarType::Int || t.scalar_type() == at::ScalarType::Long, name,
              " must have dtype torch.int32 or torch.int64");
  return t.scalar_type() == at::ScalarType::Long ? HIF8_INDEX_INT64 : HIF8_INDEX_INT32;
}

void CheckCache(const at::Tensor &cache, const char *name, int64_t heads, int64_t width) {
  CheckContiguousDevice(cache, name);
  TORCH_CHECK(cache.scalar_type() == at::ScalarType::Byte, name, " must have dtype torch.uint8");
  TORCH_CHECK(cache.dim() == 4, name, " must have shape [num_blocks, block_size, num_kv_heads, head_size + 4]");
  CheckPositiveDimensions(cache, name);
  TORCH_CHECK(cache.size(2) == heads, name, " has ", cache.size(2), " KV heads, expected ", heads);
  TORCH_CHECK(cache.size(3) == width, name, " row width must be ", width, ", got ", cache.size(3));
}

void Hif8KVCacheWrite(const at::Tensor &key, const at::Tensor &value, const at::Tensor &key_cache,
                      const at::Tensor &value_cache, const at::Tensor &slot_mapping, const at::Tensor &key_scale,
                      const at::Tensor &value_scale, const c10::optional<at::Tensor> &invalid_slots) {
  CheckContiguousDevice(key, "key");
  CheckContiguousDevice(value, "value");
  TORCH_CHECK(key.scalar_type() == at::ScalarType::Half || key.scalar_type() == at::ScalarType::BFloat16,
              "key must have dtype torch.float16 or torch.bfloat16");
  TORCH_CHECK(value.scalar_type() == key.scalar_type(), "value must have the dtype of key");
  TORCH_CHECK(key.dim() == 3 && value.dim() == 3, "key/value must have shape [tokens, num_kv_heads, head_size]");
  TORCH_CHECK(value.size(0) == key.size(0) && value.size(1) == key.size(1),
              "key and value must have the same token and head counts");
  const int64_t tokens = key.size(0), heads = key.size(1), d = key.size(2), dv = value.size(2);
  TORCH_CHECK(heads > 0 && d > 0 && dv > 0, "key/value dimensions must be positive");
  TORCH_CHECK(d % 4 == 0 && dv % 4 == 0, "HIF8 KV head sizes must be divisible by four so the inline FP32 scale is aligned");
  CheckCache(key_cache, "key_cache", heads, d + 4);
  CheckCache(value_cache, "value_cache", heads, dv + 4);
  TORCH_CHECK(value_cache.size(0) == key_cache.size(0) && value_cache.size(1) == key_cache.size(1),
              "key_cache and value_cache must have the same blocks");
  CheckContiguousDevice(slot_mapping, "slot_mapping");
  const int slot_code = IndexCode(slot_mapping, "slot_mapping");
  TORCH_CHECK(slot_mapping.dim() == 1 && slot_mapping.numel() == tokens, "slot_mapping must contain one slot per token");
  for (const auto *t : {&key_scale, &value_scale}) {
    CheckContiguousDevice(*t, "KV scale");
    TORCH_CHECK(t->scalar_type() == at::ScalarType::Float, "KV scales must have dtype torch.float32");
    TORCH_CHECK(t->dim() == 1 && t->numel() == heads, "KV scales must have shape [num_kv_heads]");
  }
  const auto device = key.device();
  for (const auto *t : {&value, &key_cache, &value_cache, &slot_mapping, &key_scale, &value_scale})
    CheckSameDevice(*t, device, "KV operand");
  int32_t *invalid = nullptr;
  if (invalid_slots.has_value()) {
    CheckContiguousDevice(*invalid_slots, "invalid_slots");
    TORCH_CHECK(invalid_slots->scalar_type() == at::ScalarType::Int && invalid_slots->numel() >= 1,
                "invalid_slots must be an int32 tensor with at least one element");
    CheckSameDevice(*invalid_slots, device, "invalid_slots");
    invalid = invalid_slots->data_ptr<int32_t>();
  }
  if (tokens == 0) return;
  const c10::OptionalDeviceGuard guard(device);
  CheckStatus(hif8_kv_cache_write(key.data_ptr(), value.data_ptr(), DtypeCode(key.scalar_type()), tokens, heads, d, dv,
                                  key_scale.data_ptr<float>(), value_scale.data_ptr<float>(), slot_mapping.data_ptr(),
                                  slot_code, key_cache.data_ptr<uint8_t>(), value_cache.data_ptr<uint8_t>(),
                                  key_cache.size(0), key_cache.size(1), invalid, CurrentStream(device)),
              "hif8_kv_cache_write");
}

at::Tensor Hif8PagedDecodeAttention(const at::Tensor &query, const at::Tensor &key_cache, const at::Tensor &value_cache,
                                    const at::Tensor &block_table, const at::Tensor &seq_lens, double scale,
                                    int64_t max_seq_len) {
  CheckContiguousDevice(query, "query");
  TORCH_CHECK(query.scalar_type() == at::ScalarType::Half || query.scalar_type() == at::ScalarType::BFloat16,
              "query must have dtype torch.float16 or torch.bfloat16");
  TORCH_CHECK(query.dim() == 3, "query must have shape [batch, num_heads, head_size]");
  const int64_t batch = query.size(0), heads = query.size(1), d = query.size(2);
  TORCH_CHECK(heads > 0 && d > 0, "query dimensions must be positive");
  TORCH_CHECK(key_cache.dim() == 4 && value_cache.dim() == 4, "caches must have shape [num_blocks, block_size, num_kv_heads, width]");
  const int64_t kv_heads = key_cache.size(2), dv = value_cache.size(3) - 4;
  CheckCache(key_cache, "key_cache", kv_heads, d + 4);
  CheckCache(value_cache, "value_cache", kv_heads, dv + 4);
  TORCH_CHECK(dv > 0, "value_cache rows are too short");
  TORCH_CHECK(value_cache.size(0) == key_cache.size(0) && value_cache.size(1) == key_cache.size(1),
              "key_cache and value_cache must have the same blocks");
  TORCH_CHECK(heads % kv_heads == 0, "num_heads must be divisible by num_kv_heads");
  CheckContiguousDevice(block_table, "block_table");
  const int bt_code = IndexCode(block_table, "block_table");
  TORCH_CHECK(block_table.dim() == 2 && block_table.size(0) >= batch && block_table.size(1) > 0,
              "block_table must have shape [batch, max_blocks]");
  CheckContiguousDevice(seq_lens, "seq_lens");
  TORCH_CHECK(seq_lens.scalar_type() == at::ScalarType::Int, "seq_lens must have dtype torch.int32");
  TORCH_CHECK(seq_lens.dim() == 1 && seq_lens.numel() >= batch, "seq_lens must contain one length per request");
  const int64_t block_size = key_cache.size(1);
  TORCH_CHECK(max_seq_len >= 0 && max_seq_len <= block_table.size(1) * block_size,
              "max_seq_len must be within the block table capacity");
  const auto device = query.device();
  for (const auto *t : {&key_cache, &value_cache, &block_table, &seq_lens}) CheckSameDevice(*t, device, "attention operand");
  const c10::OptionalDeviceGuard guard(device);
  auto out = at::empty({batch, heads, dv}, query.options());
  if (batch == 0) return out;
  const size_t ws_bytes =
      hif8_paged_decode_attention_workspace_size(batch, heads, kv_heads, d, dv, max_seq_len > 0 ? max_seq_len : 1);
  at::Tensor workspace;
  if (ws_bytes) workspace = at::empty({int64_t(ws_bytes)}, query.options().dtype(at::ScalarType::Byte));
  CheckStatus(hif8_paged_decode_attention(query.data_ptr(), DtypeCode(query.scalar_type()), key_cache.data_ptr<uint8_t>(),
                                          value_cache.data_ptr<uint8_t>(), key_cache.size(0), block_size, kv_heads, d, dv,
                                          block_table.data_ptr(), bt_code, block_table.size(1),
                                          seq_lens.data_ptr<int32_t>(), batch, heads, max_seq_len, float(scale),
                                          out.data_ptr(), ws_bytes ? workspace.data_ptr() : nullptr, ws_bytes,
                                          CurrentStream(device)),
              "hif8_paged_decode_attention");
  return out;
}

// Several query tokens per request (kv_runtime.py:1470-1563, TND layout):
// query [T, Hq, D], query_start_loc [batch + 1] int32, seq_lens [batch] int32
// -> [T, Hq, Dv]; rows past query_start_loc[batch] are left unwritten.
at::Tensor Hif8PagedPrefillAttention(const at::Tensor &query, const at::Tensor &key_cache,
                                     const at::Tensor &value_cache, const at::Tensor &block_table,
                                     const at::Tensor &query_start_loc, const at::Tensor &seq_lens, double scale,
                                     int64_t max_query_len, int64_t max_seq_len, bool causal) {
  CheckContiguousDevice(query, "query");
  TORCH_CHECK(query.scalar_type() == at::ScalarType::Half || query.scalar_type() == at::ScalarType::BFloat16,
              "query must have dtype torch.float16 or torch.bfloat16");
  TORCH_CHECK(query.dim() == 3, "query must have shape [tokens, num_heads, head_size]");
  const int64_t tokens = query.size(0), heads = query.size(1), d = query.size(2);
  TORCH_CHECK(heads > 0 && d > 0, "query dimensions must be positive");
  TORCH_CHECK(key_cache.dim() == 4 && value_cache.dim() == 4,
              "caches must have shape [num_blocks, block_size, num_kv_heads, width]");
  const int64_t kv_heads = key_cache.size(2), dv = value_cache.size(3) - 4;
  CheckCache(key_cache, "key_cache", kv_heads, d + 4);
  CheckCache(value_cache, "value_cache", kv_heads, dv + 4);
  TORCH_CHECK(dv > 0, "value_cache rows are too short");
  TORCH_CHECK(value_cache.size(0) == key_cache.size(0) && value_cache.size(1) == key_cache.size(1),
              "key_cache and value_cache must have the same blocks");
  TORCH_CHECK(heads % kv_heads == 0, "num_heads must be divisible by num_kv_heads");
  CheckContiguousDevice(query_start_loc, "query_start_loc");
  TORCH_CHECK(query_start_loc.scalar_type() == at::ScalarType::Int && query_start_loc.dim() == 1 &&
                  query_start_loc.numel() >= 1,
              "query_start_loc must be an int32 tensor [batch + 1]");
  const int64_t batch = query_start_loc.numel() - 1;
  CheckContiguousDevice(block_table, "block_table");
  const int bt_code = IndexCode(block_table, "block_table");
  TORCH_CHECK(block_table.dim() == 2 && block_table.size(0) >= batch && block_table.size(1) > 0,
              "block_table must have shape [batch, max_blocks]");
  CheckContiguousDevice(seq_lens, "seq_lens");
  TORCH_CHECK(seq_lens.scalar_type() == at::ScalarType::Int, "seq_lens must have dtype torch.int32");
  TORCH_CHECK(seq_lens.dim() == 1 && seq_lens.numel() >= batch, "seq_lens must contain one length per request");
  const int64_t block_size = key_cache.size(1);
  TORCH_CHECK(max_seq_len >= 0 && max_seq_len <= block_table.size(1) * block_size,
              "max_seq_len must be within the block table capacity");
  TORCH_CHECK(max_query_len >= 0, "max_query_len must be non-negative");
  const auto device = query.device();
  for (const auto *t : {&key_cache, &value_cache, &block_table, &seq_lens, &query_start_loc})
    CheckSameDevice(*t, device, "attention operand");
  const c10::OptionalDeviceGuard guard(device);
  auto out = at::empty({tokens, heads, dv}, query.options());
  if (batch == 0 || tokens == 0 || max_query_len == 0) return out;
  const size_t ws_bytes = hif8_paged_prefill_attention_workspace_size(batch, heads, kv_heads, d, dv, tokens,
                                                                      max_query_len, max_seq_len > 0 ? max_seq_len : 1);
  at::Tensor workspace;
  if (ws_bytes) workspace = at::empty({int64_t(ws_bytes)}, query.options().dtype(at::ScalarType::Byte));
  CheckStatus(hif8_paged_prefill_attention(
                  query.data_ptr(), DtypeCode(query.scalar_type()), key_cache.data_ptr<uint8_t>(),
                  value_cache.data_ptr<uint8_t>(), key_cache.size(0), block_size, kv_heads, d, dv,
                  block_table.data_ptr(), bt_code, block_table.size(1), query_start_loc.data_ptr<int32_t>(),
                  seq_lens.data_ptr<int32_t>(), batch, heads, tokens, max_query_len, max_seq_len, float(scale),
                  causal ? 1 : 0, out.data_ptr(), ws_bytes ? workspace.data_ptr() : nullptr, ws_bytes,
                  CurrentStream(device)),
              "hif8_paged_prefill_attention");
  return out;
}

// Token-embedding gather-decode (scheme.py:121-131): ids of any shape -> [*ids.shape, dim] bf16.
at::Tensor Hif8EmbeddingLookup(const at::Tensor &ids, const at::Tensor &weight, const at::Tensor &weight_scale,
                               const c10::optional<at::Tensor> &invalid_ids) {
  CheckContiguousDevice(ids, "input_ids");
  CheckContiguousDevice(weight, "weight");
  CheckContiguousDevice(weight_scale, "weight_scale");
  const int id_code = IndexCode(ids, "input_ids");
  TORCH_CHECK(weight.scalar_type() == at::ScalarType::Byte, "weight must have dtype torch.uint8");
  TORCH_CHECK(weight.dim() == 2, "weight must have shape [vocab, dim]");
  TORCH_CHECK(weight_scale.scalar_type() == at::ScalarType::Float, "weight_scale must have dtype torch.float32");
  TORCH_CHECK(weight_scale.numel() == weight.size(0), "weight_scale must contain one value per vocabulary row");
  CheckSameDevice(weight, ids.device(), "weight");
  CheckSameDevice(weight_scale, ids.device(), "weight_scale");
  std::vector<int64_t> shape(ids.sizes().begin(), ids.sizes().end());
  shape.push_back(weight.size(1));
  const c10::OptionalDeviceGuard guard(ids.device());
  auto out = at::empty(shape, weight.options().dtype(at::ScalarType::BFloat16));
  if (ids.numel() == 0) return out;
  int32_t *invalid = nullptr;
  if (invalid_ids.has_value()) {
    CheckContiguousDevice(*invalid_ids, "invalid_ids");
    TORCH_CHECK(invalid_ids->scalar_type() == at::ScalarType::Int && invalid_ids->numel() >= 1,
                "invalid_ids must be an int32 tensor with at least one element");
    invalid = invalid_ids->data_ptr<int32_t>();
  }
  CheckStatus(hif8_embedding_lookup(ids.data_ptr(), id_code, ids.numel(), weight.data_ptr<uint8_t>(),
                                    weight_scale.data_ptr<float>(), weight.size(0), weight.size(1),
                                    reinterpret_cast<uint16_t *>(out.data_ptr()), invalid,
                                    CurrentStream(ids.device())),
              "hif8_embedding_lookup");
  return out;
}

// ------------------------------------------------- synthetic-model glue

at::Tensor Hif8AddRmsNorm(at::Tensor &h, const c10::optional<at::Tensor> &delta, const at::Tensor &weight,
                          double eps) {
  CheckContiguousDevice(h, "h");
  CheckContiguousDevice(weight, "weight");
  TORCH_CHECK(h.scalar_type() == at::kBFloat16 && weight.scalar_type() == at::kBFloat16,
              "hif8_add_rms_norm takes bfloat16 tensors");
  TORCH_CHECK(h.dim() >= 1 && h.size(-1) > 0, "hif8_add_rms_norm needs rows of positive width");
  const int64_t n = h.size(-1);
  TORCH_CHECK(weight.numel() == n, "weight must have the row width");
  if (delta.has_value()) {
    CheckContiguousDevice(*delta, "delta");
    TORCH_CHECK(delta->scalar_type() == at::kBFloat16 && delta->sizes() == h.sizes(), "delta must match h");
  }
  const c10::OptionalDeviceGuard guard(h.device());
  auto out = at::empty_like(h);
  CheckStatus(hif8_add_rms_norm(reinterpret_cast<uint16_t *>(h.data_ptr()),
                                delta.has_value() ? reinterpret_cast<const uint16_t *>(delta->data_ptr()) : nullptr,
                                reinterpret_cast<const uint16_t *>(weight.data_ptr()),
                                reinterpret_cast<uint16_t *>(out.data_ptr()), h.numel() / n, n, float(eps),
                                CurrentStream(h.device())),
              "hif8_add_rms_norm");
  return out;
}

at::Tensor Hif8SiluMul(const at::Tensor &gate_up) {
  CheckContiguousDevice(gate_up, "gate_up");
  TORCH_CHECK(gate_up.scalar_type() == at::kBFloat16, "hif8_silu_mul takes bfloat16");
  TORCH_CHECK(gate_up.dim() >= 1 && gate_up.size(-1) > 0 && gate_up.size(-1) % 2 == 0,
              "gate_up width must be even and positive");
  const int64_t n = gate_up.size(-1) / 2;
  std::vector<int64_t> shape(gate_up.sizes().begin(), gate_up.sizes().end());
  shape.back() = n;
  const c10::OptionalDeviceGuard guard(gate_up.device());
  auto out = at::empty(shape, gate_up.options());
  CheckStatus(hif8_silu_mul(reinterpret_cast<const uint16_t *>(gate_up.data_ptr()),
                            reinterpret_cast<uint16_t *>(out.data_ptr()), gate_up.numel() / (2 * n), n,
                            CurrentStream(gate_up.device())),
              "hif8_silu_mul");
  return out;
}

// The fused static input quant of the two glue ops above: codes and row
// scales as hif8_static_quant gives them for the bf16 result.
void CheckInputScale(const at::Tensor &input_scale, const at::Tensor &like) {
  CheckContiguousDevice(input_scale, "input_scale");
  TORCH_CHECK(input_scale.scalar_type() == at::kFloat && input_scale.numel() == 1,
              "input_scale must be one float32 value");
  TORCH_CHECK(input_scale.device() == like.device(), "input_scale must be on the tensor's device");
}

std::vector<int64_t> LeadingShape(const at::Tensor &t) {
  return std::vector<int64_t>(t.sizes().begin(), t.sizes().end() - 1);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> Hif8AddRmsNormQuant(at::Tensor &h, const c10::optional<at::Tensor> &delta,
                                                                   const at::Tensor &weight, double eps,
                                                                   const at::Tensor &input_scale) {
  CheckContiguousDevice(h, "h");
  CheckContiguousDevice(weight, "weight");
  TORCH_CHECK(h.scalar_type() == at::kBFloat16 && weight.scalar_type() == at::kBFloat16,
              "hif8_add_rms_norm_quant takes bfloat16 tensors");
  TORCH_CHECK(h.dim() >= 1 && h.size(-1) > 0, "hif8_add_rms_norm_quant needs rows of positive width");
  const int64_t n = h.size(-1);
  TORCH_CHECK(weight.numel() == n, "weight must have the row width");
  if (delta.has_value()) {
    CheckContiguousDevice(*delta, "delta");
    TORCH_CHECK(delta->scalar_type() == at::kBFloat16 && delta->sizes() == h.sizes(), "delta must match h");
  }
  CheckInputScale(input_scale, h);
  const c10::OptionalDeviceGuard guard(h.device());
  auto out = at::empty_like(h);
  auto codes = at::empty(h.sizes(), h.options().dtype(at::kByte));
  auto row_scale = at::empty(LeadingShape(h), h.options().dtype(at::kFloat));
  CheckStatus(hif8_add_rms_norm_quant(
                  reinterpret_cast<uint16_t *>(h.data_ptr()),
                  delta.has_value() ? reinterpret_cast<const uint16_t *>(delta->data_ptr()) : nullptr,
                  reinterpret_cast<const uint16_t *>(weight.data_ptr()), reinterpret_cast<uint16_t *>(out.data_ptr()),
                  input_scale.data_ptr<float>(), codes.data_ptr<uint8_t>(), row_scale.data_ptr<float>(),
                  h.numel() / n, n, float(eps), CurrentStream(h.device())),
              "hif8_add_rms_norm_quant");
  return {out, codes, row_scale};
}

std::tuple<at::Tensor, at::Tensor> Hif8SiluMulQuant(const at::Tensor &gate_up, const at::Tensor &input_scale) {
  CheckContiguousDevice(gate_up, "gate_up");
  TORCH_CHECK(gate_up.scalar_type() == at::kBFloat16, "hif8_silu_mul_quant takes bfloat16");
  TORCH_CHECK(gate_up.dim() >= 1 && gate_up.size(-1) > 0 && gate_up.size(-1) % 2 == 0,
              "gate_up width must be even and positive");
  CheckInputScale(input_scale, gate_up);
  const int64_t n = gate_up.size(-1) / 2;
  std::vector<int64_t> shape(gate_up.sizes().begin(), gate_up.sizes().end());
  shape.back() = n;
  const c10::OptionalDeviceGuard guard(gate_up.device());
  auto codes = at::empty(shape, gate_up.options().dtype(at::kByte));
  auto row_scale = at::empty(LeadingShape(gate_up), gate_up.options().dtype(at::kFloat));
  CheckStatus(hif8_silu_mul_quant(reinterpret_cast<const uint16_t *>(gate_up.data_ptr()), input_scale.data_ptr<float>(),
                                  codes.data_ptr<uint8_t>(), row_scale.data_ptr<float>(), gate_up.numel() / (2 * n), n,
                                  CurrentStream(gate_up.device())),
              "hif8_silu_mul_quant");
  return {codes, row_scale};
}

// The gate_up projection over activation codes fused with SiLU-mul and the
// down projection's static input quant (no reference counterpart); where the
// fused GEMV does not take the shape, soft_hif8_gemm + hif8_silu_mul_quant.
std::tuple<at::Tensor, at::Tensor> Hif8GateUpSiluMulQuant(const at::Tensor &activation, const at::Tensor &weight,
                                                          const at::Tensor &token_scale,
                                                          const at::Tensor &channel_scale,
                                                          const at::Tensor &input_scale) {
  ValidateSoftLinear(activation, weight, token_scale, channel_scale, c10::nullopt, at::ScalarType::BFloat16, false);
  TORCH_CHECK(weight.size(0) % 2 == 0, "hif8_gate_up_silu_mul_quant needs an even number of weight rows");
  CheckContiguousDevice(input_scale, "input_scale");
  TORCH_CHECK(input_scale.scalar_type() == at::kFloat && input_scale.numel() == 1,
              "input_scale must be one float32 value");
  const c10::OptionalDeviceGuard guard(activation.device());
  const int64_t m = activation.size(0), inter = weight.size(0) / 2, k = activation.size(1);
  auto codes = at::empty({m, inter}, activation.options());
  auto row_scale = at::empty({m}, activation.options().dtype(at::kFloat));
  const int st = hif8_gate_up_silu_mul_quant(activation.data_ptr<uint8_t>(), weight.data_ptr<uint8_t>(),
                                             token_scale.data_ptr<float>(), channel_scale.data_ptr<float>(),
                                             input_scale.data_ptr<float>(), codes.data_ptr<uint8_t>(),
                                             row_scale.data_ptr<float>(), m, inter, k,
                                             CurrentStream(activation.device()));
  if (st != HIF8_ERR_UNSUPPORTED) {
    CheckStatus(st, "hif8_gate_up_silu_mul_quant");
    return {codes, row_scale};
  }
  return Hif8SiluMulQuant(SoftHif8Gemm(activation, weight, token_scale, channel_scale, c10::nullopt,
                                       at::ScalarType::BFloat16),
                          input_scale);
}

// The qkvz projection over activation codes with the linear-attention causal
// conv in its epilogue (no reference counterpart): (bf16 projection [m, n],
// float32 conv outputs [m, channels]), conv_state shifted in place.
std::tuple<at::Tensor, at::Tensor> Hif8LinearConv(const at::Tensor &activation, const at::Tensor &weight,
                                                  const at::Tensor &token_scale, const at::Tensor &channel_scale,
                                                  const at::Tensor &conv_weight, at::Tensor &conv_state) {
  ValidateSoftLinear(activation, weight, token_scale, channel_scale, c10::nullopt, at::ScalarType::BFloat16, false);
  CheckContiguousDevice(conv_weight, "conv_weight");
  CheckContiguousDevice(conv_state, "conv_state");
  TORCH_CHECK(conv_weight.scalar_type() == at::kBFloat16 && conv_state.scalar_type() == at::kBFloat16,
              "hif8_linear_conv takes bfloat16 conv_weight and conv_state");
  const int64_t m = activation.size(0), n = weight.size(0), k = activation.size(1);
  TORCH_CHECK(conv_weight.dim() == 2 && conv_weight.size(0) > 0 && conv_weight.size(0) <= n &&
                  conv_weight.size(1) >= 2 && conv_weight.size(1) <= 4,
              "hif8_linear_conv needs conv_weight [channels <= n, 2 <= conv_width <= 4]");
  const int64_t channels = conv_weight.size(0), kw = conv_weight.size(1);
  TORCH_CHECK(conv_state.dim() == 3 && conv_state.size(0) == m && conv_state.size(1) == channels &&
                  conv_state.size(2) == kw - 1,
              "hif8_linear_conv needs conv_state [m, channels, conv_width - 1]");
  const c10::OptionalDeviceGuard guard(activation.device());
  auto out = at::empty({m, n}, activation.options().dtype(at::kBFloat16));
  auto conv = at::empty({m, channels}, activation.options().dtype(at::kFloat));
  CheckStatus(hif8_linear_conv(activation.data_ptr<uint8_t>(), weight.data_ptr<uint8_t>(),
                               token_scale.data_ptr<float>(), channel_scale.data_ptr<float>(),
                               reinterpret_cast<uint16_t *>(out.data_ptr()),
                               reinterpret_cast<const uint16_t *>(conv_weight.data_ptr()),
                               reinterpret_cast<uint16_t *>(conv_state.data_ptr()), conv.data_ptr<float>(), m, n, k,
                               channels, kw, CurrentStream(activation.device())),
              "hif8_linear_conv");
  return {out, conv};
}

at::Tensor Hif8Bf16Gemv(const at::Tensor &x, const at::Tensor &weight) {
  CheckContiguousDevice(x, "x");
  CheckContiguousDevice(weight, "weight");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16 && weight.scalar_type() == at::kBFloat16,
              "hif8_bf16_gemv takes bfloat16 x and weight");
  TORCH_CHECK(x.dim() == 2 && weight.dim() == 2 && x.size(1) == weight.size(1),
              "hif8_bf16_gemv needs x [M, K] and weight [N, K]");
  const c10::OptionalDeviceGuard guard(x.device());
  auto out = at::empty({x.size(0), weight.size(0)}, x.options());
  CheckStatus(hif8_bf16_gemv(reinterpret_cast<const uint16_t *>(x.data_ptr()),
                             reinterpret_cast<const uint16_t *>(weight.data_ptr()),
                             reinterpret_cast<uint16_t *>(out.data_ptr()), x.size(0), weight.size(0), x.size(1),
                             CurrentStream(x.device())),
              "hif8_bf16_gemv");
  return out;
}

at::Tensor Hif8GdnDecodeStep(const at::Tensor &mixed, const at::Tensor &ba, const at::Tensor &conv_weight,
                             at::Tensor &conv_state, const at::Tensor &a_log, const at::Tensor &dt_bias,
                             at::Tensor &rec_state, const at::Tensor &out_norm, int64_t k_heads, int64_t v_heads,
                             int64_t k_dim, int64_t v_dim, double eps) {
  for (auto *t : {&mixed, &ba, &conv_weight, &a_log, &dt_bias, &out_norm}) CheckContiguousDevice(*t, "operand");
  CheckContiguousDevice(conv_state, "conv_state");
  CheckContiguousDevice(rec_state, "rec_state");
  TORCH_CHECK(mixed.dim() == 2 && ba.dim() == 2 && conv_weight.dim() == 2 && conv_state.dim() == 3 &&
                  rec_state.dim() == 4, "hif8_gdn_decode_step: operand ranks");
  const int64_t batch = mixed.size(0);
  const int64_t channels = 2 * k_heads * k_dim + v_heads * v_dim;
  TORCH_CHECK(mixed.scalar_type() == at::kBFloat16 && ba.scalar_type() == at::kBFloat16 &&
                  conv_weight.scalar_type() == at::kBFloat16 && conv_state.scalar_type() == at::kBFloat16 &&
                  out_norm.scalar_type() == at::kBFloat16,
              "hif8_gdn_decode_step: bf16 operands expected");
  TORCH_CHECK(a_log.scalar_type() == at::kFloat && dt_bias.scalar_type() == at::kFloat &&
                  rec_state.scalar_type() == at::kFloat, "hif8_gdn_decode_step: float32 a_log / dt_bias / state");
  TORCH_CHECK(ba.size(0) == batch && ba.size(1) == 2 * v_heads, "ba must be [batch, 2 v_heads]");
  TORCH_CHECK(conv_weight.size(0) == channels && conv_state.size(0) == batch && conv_state.size(1) == channels &&
                  conv_state.size(2) == conv_weight.size(1) - 1, "conv weight / state shapes");
  TORCH_CHECK(rec_state.size(0) == batch && rec_state.size(1) == v_heads && rec_state.size(2) == k_dim &&
                  rec_state.size(3) == v_dim, "rec_state must be [batch, v_heads, k_dim, v_dim]");
  TORCH_CHECK(a_log.numel() == v_heads && dt_bias.numel() == v_heads && out_norm.numel() == v_dim,
              "per-head parameters");
  const c10::OptionalDeviceGuard guard(mixed.device());
  auto out = at::empty({batch, v_heads * v_dim}, mixed.options());
  auto scratch = at::empty({batch, channels}, mixed.options().dtype(at::kFloat));
  CheckStatus(hif8_gdn_decode_step(
                  reinterpret_cast<const uint16_t *>(mixed.data_ptr()), mixed.size(1),
                  reinterpret_cast<const uint16_t *>(ba.data_ptr()),
                  reinterpret_cast<const uint16_t *>(conv_weight.data_ptr()),
                  reinterpret_cast<uint16_t *>(conv_state.data_ptr()), a_log.data_ptr<float>(),
                  dt_bias.data_ptr<float>(), rec_state.data_ptr<float>(),
                  reinterpret_cast<const uint16_t *>(out_norm.data_ptr()), reinterpret_cast<uint16_t *>(out.data_ptr()),
                  scratch.data_ptr<float>(), batch, k_heads, v_heads, k_dim, v_dim, conv_weight.size(1), float(eps),
                  CurrentStream(mixed.device())),
              "hif8_gdn_decode_step");
  return out;
}

// The recurrence of one decode token from hif8_linear_conv's conv outputs,
// the b/a projection of x folded in, one block per (request, value head).
at::Tensor Hif8GdnDecodeHead(const at::Tensor &conv, const at::Tensor &mixed, const at::Tensor &x,
                             const at::Tensor &ba_weight, const at::Tensor &a_log, const at::Tensor &dt_bias,
                             at::Tensor &rec_state, const at::Tensor &out_norm, int64_t k_heads, int64_t v_heads,
                             int64_t k_dim, int64_t v_dim, double eps) {
  for (auto *t : {&conv, &mixed, &x, &ba_weight, &a_log, &dt_bias, &out_norm}) CheckContiguousDevice(*t, "operand");
  CheckContiguousDevice(rec_state, "rec_state");
  TORCH_CHECK(conv.dim() == 2 && mixed.dim() == 2 && x.dim() == 2 && ba_weight.dim() == 2 && rec_state.dim() == 4,
              "hif8_gdn_decode_head: operand ranks");
  const int64_t batch = conv.size(0);
  const int64_t channels = 2 * k_heads * k_dim + v_heads * v_dim;
  TORCH_CHECK(conv.scalar_type() == at::kFloat && conv.size(1) == channels,
              "hif8_gdn_decode_head needs float32 conv [batch, 2 k_heads k_dim + v_heads v_dim]");
  TORCH_CHECK(mixed.scalar_type() == at::kBFloat16 && x.scalar_type() == at::kBFloat16 &&
                  ba_weight.scalar_type() == at::kBFloat16 && out_norm.scalar_type() == at::kBFloat16,
              "hif8_gdn_decode_head: bf16 mixed_qkvz / x / ba_weight / out_norm expected");
  TORCH_CHECK(mixed.size(0) == batch && x.size(0) == batch && x.size(1) == ba_weight.size(1) &&
                  ba_weight.size(0) == 2 * v_heads,
              "hif8_gdn_decode_head needs mixed_qkvz [batch, .], x [batch, hidden], ba_weight [2 v_heads, hidden]");
  TORCH_CHECK(a_log.scalar_type() == at::kFloat && dt_bias.scalar_type() == at::kFloat &&
                  rec_state.scalar_type() == at::kFloat, "hif8_gdn_decode_head: float32 a_log / dt_bias / state");
  TORCH_CHECK(rec_state.size(0) == batch && rec_state.size(1) == v_heads && rec_state.size(2) == k_dim &&
                  rec_state.size(3) == v_dim, "rec_state must be [batch, v_heads, k_dim, v_dim]");
  TORCH_CHECK(a_log.numel() == v_heads && dt_bias.numel() == v_heads && out_norm.numel() == v_dim,
              "per-head parameters");
  const c10::OptionalDeviceGuard guard(conv.device());
  auto out = at::empty({batch, v_heads * v_dim}, mixed.options());
  CheckStatus(hif8_gdn_decode_head(conv.data_ptr<float>(), reinterpret_cast<const uint16_t *>(mixed.data_ptr()),
                                   mixed.size(1), reinterpret_cast<const uint16_t *>(x.data_ptr()),
                                   reinterpret_cast<const uint16_t *>(ba_weight.data_ptr()), x.size(1),
                                   a_log.data_ptr<float>(), dt_bias.data_ptr<float>(), rec_state.data_ptr<float>(),
                                   reinterpret_cast<const uint16_t *>(out_norm.data_ptr()),
                                   reinterpret_cast<uint16_t *>(out.data_ptr()), batch, k_heads, v_heads, k_dim,
                                   v_dim, float(eps), CurrentStream(conv.device())),
              "hif8_gdn_decode_head");
  return out;
}

// hif8_gdn_decode_step with the b/a projection of x folded in; shapes the
// fused kernel does not take run hif8_bf16_gemv + hif8_gdn_decode_step.
at::Tensor Hif8GdnDecodeToken(const at::Tensor &mixed, const at::Tensor &x, const at::Tensor &ba_weight,
                              const at::Tensor &conv_weight, at::Tensor &conv_state, const at::Tensor &a_log,
                              const at::Tensor &dt_bias, at::Tensor &rec_state, const at::Tensor &out_norm,
                              int64_t k_heads, int64_t v_heads, int64_t k_dim, int64_t v_dim, double eps) {
  CheckContiguousDevice(x, "x");
  CheckContiguousDevice(ba_weight, "ba_weight");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16 && ba_weight.scalar_type() == at::kBFloat16,
              "hif8_gdn_decode_token takes bfloat16 x and ba_weight");
  TORCH_CHECK(x.dim() == 2 && ba_weight.dim() == 2 && x.size(0) == mixed.size(0) && x.size(1) == ba_weight.size(1) &&
                  ba_weight.size(0) == 2 * v_heads,
              "hif8_gdn_decode_token needs x [batch, hidden] and ba_weight [2 v_heads, hidden]");
  for (auto *t : {&mixed, &conv_weight, &a_log, &dt_bias, &out_norm}) CheckContiguousDevice(*t, "operand");
  CheckContiguousDevice(conv_state, "conv_state");
  CheckContiguousDevice(rec_state, "rec_state");
  TORCH_CHECK(mixed.dim() == 2 && conv_weight.dim() == 2 && conv_state.dim() == 3 && rec_state.dim() == 4,
              "hif8_gdn_decode_token: operand ranks");
  const int64_t batch = mixed.size(0);
  const int64_t channels = 2 * k_heads * k_dim + v_heads * v_dim;
  TORCH_CHECK(mixed.scalar_type() == at::kBFloat16 && conv_weight.scalar_type() == at::kBFloat16 &&
                  conv_state.scalar_type() == at::kBFloat16 && out_norm.scalar_type() == at::kBFloat16,
              "hif8_gdn_decode_token: bf16 operands expected");
  TORCH_CHECK(a_log.scalar_type() == at::kFloat && dt_bias.scalar_type() == at::kFloat &&
                  rec_state.scalar_type() == at::kFloat, "hif8_gdn_decode_token: float32 a_log / dt_bias / state");
  TORCH_CHECK(conv_weight.size(0) == channels && conv_state.size(0) == batch && conv_state.size(1) == channels &&
                  conv_state.size(2) == conv_weight.size(1) - 1, "conv weight / state shapes");
  TORCH_CHECK(rec_state.size(0) == batch && rec_state.size(1) == v_heads && rec_state.size(2) == k_dim &&
                  rec_state.size(3) == v_dim, "rec_state must be [batch, v_heads, k_dim, v_dim]");
  TORCH_CHECK(a_log.numel() == v_heads && dt_bias.numel() == v_heads && out_norm.numel() == v_dim,
              "per-head parameters");
  const c10::OptionalDeviceGuard guard(mixed.device());
  auto out = at::empty({batch, v_heads * v_dim}, mixed.options());
  const int st = hif8_gdn_decode_token(
      reinterpret_cast<const uint16_t *>(mixed.data_ptr()), mixed.size(1),
      reinterpret_cast<const uint16_t *>(x.data_ptr()), reinterpret_cast<const uint16_t *>(ba_weight.data_ptr()),
      x.size(1), reinterpret_cast<const uint16_t *>(conv_weight.data_ptr()),
      reinterpret_cast<uint16_t *>(conv_state.data_ptr()), a_log.data_ptr<float>(), dt_bias.data_ptr<float>(),
      rec_state.data_ptr<float>(), reinterpret_cast<const uint16_t *>(out_norm.data_ptr()),
      reinterpret_cast<uint16_t *>(out.data_ptr()), batch, k_heads, v_heads, k_dim, v_dim, conv_weight.size(1),
      float(eps), CurrentStream(mixed.device()));
  if (st != HIF8_ERR_UNSUPPORTED) {
    CheckStatus(st, "hif8_gdn_decode_token");
    return out;
  }
  const at::Tensor ba = Hif8Bf16Gemv(x, ba_weight);
  return Hif8GdnDecodeStep(mixed, ba, conv_weight, conv_state, a_log, dt_bias, rec_state, out_norm, k_heads, v_heads,
                           k_dim, v_dim, eps);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> Hif8QkNormRope(
    const at::Tensor &qkv, const at::Tensor &q_norm, const at::Tensor &k_norm, const at::Tensor &pos,
    const at::Tensor &inv_freq, const at::Tensor &block_table, int64_t block_size, int64_t num_heads,
    int64_t num_kv_heads, int64_t head_size, double eps) {
  for (auto *t : {&qkv, &q_norm, &k_norm, &pos, &inv_freq, &block_table}) CheckContiguousDevice(*t, "operand");
  TORCH_CHECK(qkv.scalar_type() == at::kBFloat16 && q_norm.scalar_type() == at::kBFloat16 &&
                  k_norm.scalar_type() == at::kBFloat16, "hif8_qk_norm_rope: bf16 qkv and norms");
  TORCH_CHECK(pos.scalar_type() == at::kLong && inv_freq.scalar_type() == at::kFloat &&
                  block_table.scalar_type() == at::kInt, "hif8_qk_norm_rope: int64 pos, float32 inv_freq, int32 table");
  const int64_t batch = qkv.size(0);
  TORCH_CHECK(qkv.numel() == batch * (num_heads + 2 * num_kv_heads) * head_size, "qkv width");
  TORCH_CHECK(pos.numel() == batch && block_table.dim() == 2 && block_table.size(0) >= batch, "pos / block_table");
  const c10::OptionalDeviceGuard guard(qkv.device());
  auto q = at::empty({batch, num_heads, head_size}, qkv.options());
  auto k = at::empty({batch, num_kv_heads, head_size}, qkv.options());
  auto v = at::empty({batch, num_kv_heads, head_size}, qkv.options());
  auto slots = at::empty({batch}, qkv.options().dtype(at::kLong));
  CheckStatus(hif8_qk_norm_rope(reinterpret_cast<const uint16_t *>(qkv.data_ptr()),
                                reinterpret_cast<const uint16_t *>(q_norm.data_ptr()),
                                reinterpret_cast<const uint16_t *>(k_norm.data_ptr()), pos.data_ptr<int64_t>(),
                                inv_freq.data_ptr<float>(), block_table.data_ptr<int32_t>(), block_table.size(1),
                                block_size, reinterpret_cast<uint16_t *>(q.data_ptr()),
                                reinterpret_cast<uint16_t *>(k.data_ptr()), reinterpret_cast<uint16_t *>(v.data_ptr()),
                                slots.data_ptr<int64_t>(), batch, num_heads, num_kv_heads, head_size,
                                2 * inv_freq.numel(), float(eps), CurrentStream(qkv.device())),
              "hif8_qk_norm_rope");
  return {q, k, v, slots};
}

// ------------------------------------------------------------------ Meta

std::tuple<at::Tensor, at::Tensor> Hif8StaticQuantMeta(const at::Tensor &x, const at::Tensor &fixed_scale) {
  (void)fixed_scale;
  auto data = at::empty_like(x, x.options().dtype(at::kByte));
  int64_t rows = 1;  // product of the leading dimensions (no division: the last may be 0)
  for (int64_t i = 0; i + 1 < x.dim(); ++i) rows *= x.size(i);
  return {data, at::empty({rows}, x.options().dtype(at::kFloat))};
}

std::tuple<at::Tensor, at::Tensor> Hif8DynamicQuantMeta(const at::Tensor &x) {
  auto data = at::empty_like(x, x.options().dtype(at::kByte));
  int64_t rows = 1;  // product of the leading dimensions (no division: the last may be 0)
  for (int64_t i = 0; i + 1 < x.dim(); ++i) rows *= x.size(i);
  return {data, at::empty({rows}, x.options().dtype(at::kFloat))};
}

at::Tensor FusedLinearMeta(const at::Tensor &activation, const at::Tensor &weight, const at::Tensor &,
                           const c10::optional<at::Tensor> &, at::ScalarType output_dtype) {
  return at::empty({activation.size(0), weight.size(0)}, activation.options().dtype(output_dtype));
}

at::Tensor Hif8DecodeBf16Meta(const at::Tensor &codes) {
  return at::empty_like(codes, codes.options().dtype(at::kBFloat16));
}

at::Tensor Hif8ScaledDecodeMeta(const at::Tensor &data, const at::Tensor &) {
  return at::empty_like(data, data.options().dtype(at::kBFloat16));
}

at::Tensor LinearMeta(const at::Tensor &activation, const at::Tensor &weight, const at::Tensor &,
                      const at::Tensor &, const c10::optional<at::Tensor> &, at::ScalarType output_dtype) {
  return at::empty({activation.size(0), weight.size(0)}, activation.options().dtype(output_dtype));
}

void Hif8KVCacheWriteMeta(const at::Tensor &, const at::Tensor &, const at::Tensor &, const at::Tensor &,
                          const at::Tensor &, const at::Tensor &, const at::Tensor &,
                          const c10::optional<at::Tensor> &) {}

at::Tensor Hif8PagedDecodeAttentionMeta(const at::Tensor &query, const at::Tensor &, const at::Tensor &value_cache,
                                        const at::Tensor &, const at::Tensor &, double, int64_t) {
  return at::empty({query.size(0), query.size(1), value_cache.size(3) - 4}, query.options());
}

at::Tensor Hif8PagedPrefillAttentionMeta(const at::Tensor &query, const at::Tensor &, const at::Tensor &value_cache,
                                         const at::Tensor &, const at::Tensor &, const at::Tensor &, double, int64_t,
                                         int64_t, bool) {
  return at::empty({query.size(0), query.size(1), value_cache.size(3) - 4}, query.options());
}

at::Tensor Hif8EmbeddingLookupMeta(const at::Tensor &ids, const at::Tensor &weight, const at::Tensor &,
                                   const c10::optional<at::Tensor> &) {
  std::vector<int64_t> shape(ids.sizes().begin(), ids.sizes().end());
  shape.push_back(weight.size(1));
  return at::empty(shape, weight.options().dtype(at::kBFloat16));
}

// The decode glue ops (shapes and dtypes of the CUDA implementations above).
at::Tensor Hif8AddRmsNormMeta(at::Tensor &h, const c10::optional<at::Tensor> &, const at::Tensor &, double) {
  return at::empty_like(h);
}

at::Tensor Hif8SiluMulMeta(const at::Tensor &gate_up) {
  std::vector<int64_t> shape(gate_up.sizes().begin(), gate_up.sizes().end());
  shape.back() /= 2;
  return at::empty(shape, gate_up.options());
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> Hif8AddRmsNormQuantMeta(at::Tensor &h, const c10::optional<at::Tensor> &,
                                                                       const at::Tensor &, double, const at::Tensor &) {
  return {at::empty_like(h), at::empty(h.sizes(), h.options().dtype(at::kByte)),
          at::empty(LeadingShape(h), h.options().dtype(at::kFloat))};
}

std::tuple<at::Tensor, at::Tensor> Hif8SiluMulQuantMeta(const at::Tensor &gate_up, const at::Tensor &) {
  std::vector<int64_t> shape(gate_up.sizes().begin(), gate_up.sizes().end());
  shape.back() /= 2;
  return {at::empty(shape, gate_up.options().dtype(at::kByte)),
          at::empty(LeadingShape(gate_up), gate_up.options().dtype(at::kFloat))};
}

at::Tensor Hif8Bf16GemvMeta(const at::Tensor &x, const at::Tensor &weight) {
  return at::empty({x.size(0), weight.size(0)}, x.options());
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> Hif8QkNormRopeMeta(
    const at::Tensor &qkv, const at::Tensor &, const at::Tensor &, const at::Tensor &, const at::Tensor &,
    const at::Tensor &, int64_t, int64_t num_heads, int64_t num_kv_heads, int64_t head_size, double) {
  const int64_t batch = qkv.size(0);
  return {at::empty({batch, num_heads, head_size}, qkv.options()),
          at::empty({batch, num_kv_heads, head_size}, qkv.options()),
          at::empty({batch, num_kv_heads, head_size}, qkv.options()),
          at::empty({batch}, qkv.options().dtype(at::kLong))};
}

at::Tensor Hif8GdnDecodeStepMeta(const at::Tensor &mixed, const at::Tensor &, const at::Tensor &, at::Tensor &,
                                 const at::Tensor &, const at::Tensor &, at::Tensor &, const at::Tensor &, int64_t,
                                 int64_t v_heads, int64_t, int64_t v_dim, double) {
  return at::empty({mixed.size(0), v_heads * v_dim}, mixed.options());
}

std::tuple<at::Tensor, at::Tensor> Hif8GateUpSiluMulQuantMeta(const at::Tensor &activation, const at::Tensor &weight,
                                                              const at::Tensor &, const at::Tensor &,
                                                              const at::Tensor &) {
  return {at::empty({activation.size(0), weight.size(0) / 2}, activation.options()),
          at::empty({activation.size(0)}, activation.options().dtype(at::kFloat))};
}

std::tuple<at::Tensor, at::Tensor> Hif8LinearConvMeta(const at::Tensor &activation, const at::Tensor &weight,
                                                      const at::Tensor &, const at::Tensor &,
                                                      const at::Tensor &conv_weight, at::Tensor &) {
  return {at::empty({activation.size(0), weight.size(0)}, activation.options().dtype(at::kBFloat16)),
          at::empty({activation.size(0), conv_weight.size(0)}, activation.options().dtype(at::kFloat))};
}

at::Tensor Hif8GdnDecodeHeadMeta(const at::Tensor &conv, const at::Tensor &, const at::Tensor &, const at::Tensor &,
                                 const at::Tensor &, const at::Tensor &, at::Tensor &, const at::Tensor &, int64_t,
                                 int64_t v_heads, int64_t, int64_t v_dim, double) {
  return at::empty({conv.size(0), v_heads * v_dim}, conv.options().dtype(at::kBFloat16));
}

at::Tensor Hif8GdnDecodeTokenMeta(const at::Tensor &mixed, const at::Tensor &, const at::Tensor &,
                                  const at::Tensor &, at::Tensor &, const at::Tensor &, const at::Tensor &,
                                  at::Tensor &, const at::Tensor &, int64_t, int64_t v_heads, int64_t, int64_t v_dim,
                                  double) {
  return at::empty({mixed.size(0), v_heads * v_dim}, mixed.options());
}

}  // namespace

TORCH_LIBRARY(vllm_ascend_hif8, m) {
  m.def("hif8_static_quant(Tensor x, Tensor fixed_scale) -> (Tensor, Tensor)");
  m.def("hif8_scaled_decode(Tensor data, Tensor scale) -> Tensor");
  m.def("soft_hif8_gemv(Tensor activation, Tensor weight, Tensor token_scale, Tensor channel_scale, Tensor? bias, ScalarType output_dtype) -> Tensor");
  m.def("soft_hif8_gemm(Tensor activation, Tensor weight, Tensor token_scale, Tensor channel_scale, Tensor? bias, ScalarType output_dtype) -> Tensor");
  m.def("soft_hif8_static_fused_gemm(Tensor activation, Tensor weight, Tensor fixed_scale, Tensor channel_scale, Tensor? bias, ScalarType output_dtype) -> Tensor");
  m.def("hif8_kv_cache_write(Tensor key, Tensor value, Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor slot_mapping, Tensor key_scale, Tensor value_scale, Tensor(c!)? invalid_slots=None) -> ()");
  m.def("hif8_paged_decode_attention(Tensor query, Tensor key_cache, Tensor value_cache, Tensor block_table, Tensor seq_lens, float scale, int max_seq_len) -> Tensor");
  m.def("hif8_paged_prefill_attention(Tensor query, Tensor key_cache, Tensor value_cache, Tensor block_table, Tensor query_start_loc, Tensor seq_lens, float scale, int max_query_len, int max_seq_len, bool causal=True) -> Tensor");
  m.def("hif8_embedding_lookup(Tensor input_ids, Tensor weight, Tensor weight_scale, Tensor(a!)? invalid_ids=None) -> Tensor");
  m.def("hif8_dynamic_quant(Tensor x) -> (Tensor, Tensor)");
  m.def("soft_hif8_fused_gemm(Tensor activation, Tensor weight, Tensor channel_scale, Tensor? bias, ScalarType output_dtype) -> Tensor");
  m.def("hif8_add_rms_norm(Tensor(a!) h, Tensor? delta, Tensor weight, float eps) -> Tensor");
  m.def("hif8_silu_mul(Tensor gate_up) -> Tensor");
  m.def("hif8_add_rms_norm_quant(Tensor(a!) h, Tensor? delta, Tensor weight, float eps, Tensor input_scale) -> "
        "(Tensor, Tensor, Tensor)");
  m.def("hif8_silu_mul_quant(Tensor gate_up, Tensor input_scale) -> (Tensor, Tensor)");
  m.def("hif8_bf16_gemv(Tensor x, Tensor weight) -> Tensor");
  m.def("hif8_qk_norm_rope(Tensor qkv, Tensor q_norm, Tensor k_norm, Tensor pos, Tensor inv_freq, Tensor block_table, int block_size, int num_heads, int num_kv_heads, int head_size, float eps) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("soft_hif8_gemm_decoded_weight(Tensor activation, Tensor weight_bf16, Tensor token_scale, Tensor channel_scale, Tensor? bias, ScalarType output_dtype) -> Tensor");
  m.def("hif8_decode_bf16(Tensor codes) -> Tensor");
  m.def("hif8_gdn_decode_step(Tensor mixed_qkvz, Tensor ba, Tensor conv_weight, Tensor(a!) conv_state, Tensor a_log, Tensor dt_bias, Tensor(b!) rec_state, Tensor out_norm, int k_heads, int v_heads, int k_dim, int v_dim, float eps) -> Tensor");
  m.def("hif8_gate_up_silu_mul_quant(Tensor activation, Tensor weight, Tensor token_scale, Tensor channel_scale, Tensor input_scale) -> (Tensor, Tensor)");
  m.def("hif8_gdn_decode_token(Tensor mixed_qkvz, Tensor x, Tensor ba_weight, Tensor conv_weight, Tensor(a!) conv_state, Tensor a_log, Tensor dt_bias, Tensor(b!) rec_state, Tensor out_norm, int k_heads, int v_heads, int k_dim, int v_dim, float eps) -> Tensor");
  m.def("hif8_linear_conv(Tensor activation, Tensor weight, Tensor token_scale, Tensor channel_scale, Tensor conv_weight, Tensor(a!) conv_state) -> (Tensor, Tensor)");
  m.def("hif8_gdn_decode_head(Tensor conv, Tensor mixed_qkvz, Tensor x, Tensor ba_weight, Tensor a_log, Tensor dt_bias, Tensor(a!) rec_state, Tensor out_norm, int k_heads, int v_heads, int k_dim, int v_dim, float eps) -> Tensor");
}

TORCH_LIBRARY_IMPL(vllm_ascend_hif8, CUDA, m) {
  m.impl("hif8_static_quant", &Hif8StaticQuant);
  m.impl("hif8_scaled_decode", &Hif8ScaledDecode);
  m.impl("soft_hif8_gemv", &SoftHif8Gemv);
  m.impl("soft_hif8_gemm", &SoftHif8Gemm);
  m.impl("soft_hif8_static_fused_gemm", &SoftHif8StaticFusedGemm);
  m.impl("hif8_kv_cache_write", &Hif8KVCacheWrite);
  m.impl("hif8_paged_decode_attention", &Hif8PagedDecodeAttention);
  m.impl("hif8_paged_prefill_attention", &Hif8PagedPrefillAttention);
  m.impl("hif8_embedding_lookup", &Hif8EmbeddingLookup);
  m.impl("hif8_dynamic_quant", &Hif8DynamicQuant);
  m.impl("soft_hif8_fused_gemm", &SoftHif8FusedGemm);
  m.impl("hif8_add_rms_norm", &Hif8AddRmsNorm);
  m.impl("hif8_silu_mul", &Hif8SiluMul);
  m.impl("hif8_add_rms_norm_quant", &Hif8AddRmsNormQuant);
  m.impl("hif8_silu_mul_quant", &Hif8SiluMulQuant);
  m.impl("hif8_bf16_gemv", &Hif8Bf16Gemv);
  m.impl("hif8_qk_norm_rope", &Hif8QkNormRope);
  m.impl("hif8_gdn_decode_step", &Hif8GdnDecodeStep);
  m.impl("hif8_gdn_decode_token", &Hif8GdnDecodeToken);
  m.impl("hif8_gate_up_silu_mul_quant", &Hif8GateUpSiluMulQuant);
  m.impl("hif8_linear_conv", &Hif8LinearConv);
  m.impl("hif8_gdn_decode_head", &Hif8GdnDecodeHead);
  m.impl("soft_hif8_gemm_decoded_weight", &SoftHif8GemmDecodedWeight);
  m.impl("hif8_decode_bf16", &Hif8DecodeBf16);
}

TORCH_LIBRARY_IMPL(vllm_ascend_hif8, Meta, m) {
  m.impl("hif8_static_quant", &Hif8StaticQuantMeta);
  m.impl("hif8_scaled_decode", &Hif8ScaledDecodeMeta);
  m.impl("soft_hif8_gemv", &LinearMeta);
  m.impl("soft_hif8_gemm", &LinearMeta);
  m.impl("soft_hif8_static_fused_gemm", &LinearMeta);
  m.impl("hif8_kv_cache_write", &Hif8KVCacheWriteMeta);
  m.impl("hif8_paged_decode_attention", &Hif8PagedDecodeAttentionMeta);
  m.impl("hif8_paged_prefill_attention", &Hif8PagedPrefillAttentionMeta);
  m.impl("hif8_embedding_lookup", &Hif8EmbeddingLookupMeta);
  m.impl("hif8_dynamic_quant", &Hif8DynamicQuantMeta);
  m.impl("soft_hif8_fused_gemm", &FusedLinearMeta);
  m.impl("soft_hif8_gemm_decoded_weight", &LinearMeta);
  m.impl("hif8_decode_bf16", &Hif8DecodeBf16Meta);
  m.impl("hif8_add_rms_norm", &Hif8AddRmsNormMeta);
  m.impl("hif8_silu_mul", &Hif8SiluMulMeta);
  m.impl("hif8_add_rms_norm_quant", &Hif8AddRmsNormQuantMeta);
  m.impl("hif8_silu_mul_quant", &Hif8SiluMulQuantMeta);
  m.impl("hif8_bf16_gemv", &Hif8Bf16GemvMeta);
  m.impl("hif8_qk_norm_rope", &Hif8QkNormRopeMeta);
  m.impl("hif8_gdn_decode_step", &Hif8GdnDecodeStepMeta);
  m.impl("hif8_gdn_decode_token", &Hif8GdnDecodeTokenMeta);
  m.impl("hif8_gate_up_silu_mul_quant", &Hif8GateUpSiluMulQuantMeta);
  m.impl("hif8_linear_conv", &Hif8LinearConvMeta);
  m.impl("hif8_gdn_decode_head", &Hif8GdnDecodeHeadMeta);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, module) {
  module.def("hif8_static_quant", &Hif8StaticQuant, pybind11::arg("x"), pybind11::arg("fixed_scale"));
  module.def("hif8_dynamic_quant", &Hif8DynamicQuant, pybind11::arg("x"));
  module.def("soft_hif8_fused_gemm", &SoftHif8FusedGemm, pybind11::arg("activation"), pybind11::arg("weight"),
             pybind11::arg("channel_scale"), pybind11::arg("bias") = c10::nullopt,
             pybind11::arg("output_dtype") = at::ScalarType::Half);
  module.def("hif8_scaled_decode", &Hif8ScaledDecode, pybind11::arg("data"), pybind11::arg("scale"));
  module.def("soft_hif8_gemv", &SoftHif8Gemv, pybind11::arg("activation"), pybind11::arg("weight"),
             pybind11::arg("token_scale"), pybind11::arg("channel_scale"), pybind11::arg("bias") = c10::nullopt,
             pybind11::arg("output_dtype") = at::ScalarType::Half);
  module.def("soft_hif8_gemm", &SoftHif8Gemm, pybind11::arg("activation"), pybind11::arg("weight"),
             pybind11::arg("token_scale"), pybind11::arg("channel_scale"), pybind11::arg("bias") = c10::nullopt,
             pybind11::arg("output_dtype") = at::ScalarType::Half);
  module.def("soft_hif8_static_fused_gemm", &SoftHif8StaticFusedGemm, pybind11::arg("activation"),
             pybind11::arg("weight"), pybind11::arg("fixed_scale"), pybind11::arg("channel_scale"),
             pybind11::arg("bias") = c10::nullopt, pybind11::arg("output_dtype") = at::ScalarType::Half);
  module.def("hif8_kv_cache_write", &Hif8KVCacheWrite, pybind11::arg("key"), pybind11::arg("value"),
             pybind11::arg("key_cache"), pybind11::arg("value_cache"), pybind11::arg("slot_mapping"),
             pybind11::arg("key_scale"), pybind11::arg("value_scale"), pybind11::arg("invalid_slots") = c10::nullopt);
  module.def("hif8_paged_decode_attention", &Hif8PagedDecodeAttention, pybind11::arg("query"),
             pybind11::arg("key_cache"), pybind11::arg("value_cache"), pybind11::arg("block_table"),
             pybind11::arg("seq_lens"), pybind11::arg("scale"), pybind11::arg("max_seq_len"));
}
