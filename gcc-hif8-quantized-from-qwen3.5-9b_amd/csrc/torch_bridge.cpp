// Thin torch extension over the C ABI in include/hif8_rocm.h.
//
// Registers the reference's operator schemas under the same namespace
// (pybind.cpp:6-13) so callers of torch.ops.vllm_ascend_hif8.* switch over
// unchanged, with implementations for HIP tensors (torch's "cuda" key on ROCm)
// and Meta implementations for shape inference (pybind.cpp:27-89).  Each
// implementation validates like the reference bridge (hif8_native.cpp:131-316,
// 487-611, 784-861), allocates outputs with the caching allocator and calls
// the C ABI on the current HIP stream.  No host synchronisation, no fallback.
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
                        bool gemv) {
  CheckDeviceTensor(activation, "activation");
  CheckDeviceTensor(weight, "weight");
  CheckDeviceTensor(token_scale, "token_scale");
  CheckDeviceTensor(channel_scale, "channel_scale");
  TORCH_CHECK(activation.scalar_type() == at::ScalarType::Byte, "activation must have dtype torch.uint8");
  TORCH_CHECK(weight.scalar_type() == at::ScalarType::Byte, "weight must have dtype torch.uint8");
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
  return SoftLinear(activation, weight, token_scale, channel_scale, bias, output_dtype, false, "soft_hif8_gemm",
                    &soft_hif8_gemm);
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
  CheckStatus(soft_hif8_static_fused_gemm(activation.data_ptr(), DtypeCode(activation.scalar_type()),
                                          weight.data_ptr<uint8_t>(), fixed_scale.data_ptr<float>(),
                                          channel_scale.data_ptr<float>(), bias_ptr, bias_dtype, out.data_ptr(),
                                          DtypeCode(output_dtype), activation.size(0), weight.size(0),
                                          activation.size(1), CurrentStream(device)),
              "soft_hif8_static_fused_gemm");
  return out;
}

// ------------------------------------------------------------------ Meta

std::tuple<at::Tensor, at::Tensor> Hif8StaticQuantMeta(const at::Tensor &x, const at::Tensor &fixed_scale) {
  (void)fixed_scale;
  auto data = at::empty_like(x, x.options().dtype(at::kByte));
  const int64_t rows = x.dim() ? x.numel() / x.size(-1) : 1;
  return {data, at::empty({rows}, x.options().dtype(at::kFloat))};
}

at::Tensor Hif8ScaledDecodeMeta(const at::Tensor &data, const at::Tensor &) {
  return at::empty_like(data, data.options().dtype(at::kBFloat16));
}

at::Tensor LinearMeta(const at::Tensor &activation, const at::Tensor &weight, const at::Tensor &,
                      const at::Tensor &, const c10::optional<at::Tensor> &, at::ScalarType output_dtype) {
  return at::empty({activation.size(0), weight.size(0)}, activation.options().dtype(output_dtype));
}

}  // namespace

TORCH_LIBRARY(vllm_ascend_hif8, m) {
  m.def("hif8_static_quant(Tensor x, Tensor fixed_scale) -> (Tensor, Tensor)");
  m.def("hif8_scaled_decode(Tensor data, Tensor scale) -> Tensor");
  m.def("soft_hif8_gemv(Tensor activation, Tensor weight, Tensor token_scale, Tensor channel_scale, Tensor? bias, ScalarType output_dtype) -> Tensor");
  m.def("soft_hif8_gemm(Tensor activation, Tensor weight, Tensor token_scale, Tensor channel_scale, Tensor? bias, ScalarType output_dtype) -> Tensor");
  m.def("soft_hif8_static_fused_gemm(Tensor activation, Tensor weight, Tensor fixed_scale, Tensor channel_scale, Tensor? bias, ScalarType output_dtype) -> Tensor");
}

TORCH_LIBRARY_IMPL(vllm_ascend_hif8, CUDA, m) {
  m.impl("hif8_static_quant", &Hif8StaticQuant);
  m.impl("hif8_scaled_decode", &Hif8ScaledDecode);
  m.impl("soft_hif8_gemv", &SoftHif8Gemv);
  m.impl("soft_hif8_gemm", &SoftHif8Gemm);
  m.impl("soft_hif8_static_fused_gemm", &SoftHif8StaticFusedGemm);
}

TORCH_LIBRARY_IMPL(vllm_ascend_hif8, Meta, m) {
  m.impl("hif8_static_quant", &Hif8StaticQuantMeta);
  m.impl("hif8_scaled_decode", &Hif8ScaledDecodeMeta);
  m.impl("soft_hif8_gemv", &LinearMeta);
  m.impl("soft_hif8_gemm", &LinearMeta);
  m.impl("soft_hif8_static_fused_gemm", &LinearMeta);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, module) {
  module.def("hif8_static_quant", &Hif8StaticQuant, pybind11::arg("x"), pybind11::arg("fixed_scale"));
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
}
