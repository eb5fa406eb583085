// tinyinfer_amd._C: the torch-facing wrapper over the C ABI.
//
// mlp_forward_mxfp4 keeps the reference's Python name, argument names and
// order, validation and error messages (tinyinfer/csrc/bind.cpp:656-792,
// registration :871-882), so Qwen3MLP.forward can call it unchanged. Two
// reference-only limits are dropped: N <= 65535 (a gridDim.y artefact of the
// per-token kernels, :738) and the N > 32 performance warning (:735-737).
//
// Test/bench helpers with no reference counterpart: mlp_forward_mxfp4_path
// (forced kernel path), mxfp4_dequant, mxfp4_quantize.  Fusions beyond the
// reference's call: mlp_forward_mxfp4_residual (the decoder layer's residual
// add in the down epilogue), mlp_forward_mxfp4_rmsnorm (also the
// post-attention RMSNorm in the prologue) and mxfp4_linear (MXFP4 weights for
// any linear).  rmsnorm_forward mirrors the reference's op of that name.
#include <torch/extension.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>

#include <string>

#include "../../include/tinyinfer_mxfp4.h"

namespace {

// torch on ROCm exposes HIP devices and streams under the "cuda" device type;
// this is the stream torch.cuda.current_stream() names.
void* current_stream() {
  return static_cast<void*>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
}

void check_status(int st, const char* what) {
  TORCH_CHECK(st == TI_OK, what, " failed: ", tinyinfer_mxfp4_status_string(st), " (status ", st, ")");
}

// Validation of the seven MLP inputs, in the reference's order and wording.
void check_mlp_inputs(const torch::Tensor& X, const torch::Tensor& gate, const torch::Tensor& gate_scale,
                      const torch::Tensor& up, const torch::Tensor& up_scale, const torch::Tensor& down,
                      const torch::Tensor& down_scale) {
  const std::pair<const torch::Tensor*, const char*> all[] = {
      {&X, "X"},   {&gate, "gate"}, {&gate_scale, "gate_scale"}, {&up, "up"},
      {&up_scale, "up_scale"}, {&down, "down"}, {&down_scale, "down_scale"}};
  for (const auto& t : all) TORCH_CHECK(t.first->is_cuda(), t.second, " must be a CUDA tensor");
  for (size_t i = 1; i < 7; ++i)
    TORCH_CHECK(X.device() == all[i].first->device(), "X/", all[i].second, " device mismatch");

  TORCH_CHECK(X.dim() == 2, "X must be [N, hidden_dim]");
  for (size_t i = 1; i < 7; ++i) TORCH_CHECK(all[i].first->dim() == 2, all[i].second, " must be 2D");

  const int64_t N = X.size(0);
  const int64_t hidden = X.size(1);
  const int64_t inter = gate.size(0);
  TORCH_CHECK(N > 0, "N must be positive");
  TORCH_CHECK(hidden > 0, "hidden_dim must be positive");
  TORCH_CHECK(inter > 0, "intermediate must be positive");
  TORCH_CHECK(hidden % 32 == 0, "hidden_dim must be divisible by 32");
  TORCH_CHECK(inter % 32 == 0, "intermediate must be divisible by 32");

  TORCH_CHECK(gate.size(1) == hidden / 2, "gate shape mismatch");
  TORCH_CHECK(up.size(0) == inter && up.size(1) == hidden / 2, "up shape mismatch");
  TORCH_CHECK(down.size(0) == hidden && down.size(1) == inter / 2, "down shape mismatch");
  TORCH_CHECK(gate_scale.size(0) == inter && gate_scale.size(1) == hidden / 32, "gate_scale shape mismatch");
  TORCH_CHECK(up_scale.size(0) == inter && up_scale.size(1) == hidden / 32, "up_scale shape mismatch");
  TORCH_CHECK(down_scale.size(0) == hidden && down_scale.size(1) == inter / 32, "down_scale shape mismatch");

  bool bytes = true;
  for (size_t i = 1; i < 7; ++i) bytes = bytes && all[i].first->scalar_type() == at::kByte;
  TORCH_CHECK(bytes, "MXFP4 weights and scales must be uint8");
  TORCH_CHECK(X.scalar_type() == at::kHalf || X.scalar_type() == at::kBFloat16,
              "MXFP4 MLP only supports FP16 and BF16 activations");
  for (const auto& t : all) TORCH_CHECK(t.first->is_contiguous(), t.second, " must be contiguous");
}

torch::Tensor mlp_impl(const torch::Tensor& X, const torch::Tensor& gate, const torch::Tensor& gate_scale,
                       const torch::Tensor& up, const torch::Tensor& up_scale, const torch::Tensor& down,
                       const torch::Tensor& down_scale, int path) {
  check_mlp_inputs(X, gate, gate_scale, up, up_scale, down, down_scale);
  const int64_t N = X.size(0), hidden = X.size(1), inter = gate.size(0);
  const int dtype = X.scalar_type() == at::kHalf ? TI_DTYPE_F16 : TI_DTYPE_BF16;

  c10::DeviceGuard guard(X.device());
  auto O = torch::empty({N, hidden}, X.options());
  auto tmp = torch::empty({N, inter}, X.options());  // SiLU(g)*u, caching allocator
  const int st = tinyinfer_mlp_forward_mxfp4_path(
      X.data_ptr(), gate.data_ptr<uint8_t>(), gate_scale.data_ptr<uint8_t>(), up.data_ptr<uint8_t>(),
      up_scale.data_ptr<uint8_t>(), down.data_ptr<uint8_t>(), down_scale.data_ptr<uint8_t>(),
      (size_t)N, (size_t)hidden, (size_t)inter, tmp.data_ptr(), O.data_ptr(), dtype, path,
      current_stream());
  check_status(st, "mlp_forward_mxfp4");
  return O;
}

torch::Tensor mlp_forward_mxfp4(torch::Tensor X, torch::Tensor gate, torch::Tensor gate_scale,
                                torch::Tensor up, torch::Tensor up_scale, torch::Tensor down,
                                torch::Tensor down_scale) {
  return mlp_impl(X, gate, gate_scale, up, up_scale, down, down_scale, TI_PATH_AUTO);
}

torch::Tensor mlp_forward_mxfp4_path(torch::Tensor X, torch::Tensor gate, torch::Tensor gate_scale,
                                     torch::Tensor up, torch::Tensor up_scale, torch::Tensor down,
                                     torch::Tensor down_scale, int64_t path) {
  return mlp_impl(X, gate, gate_scale, up, up_scale, down, down_scale, (int)path);
}

// residual + MLP(X), the residual add fused into the down stage
// (tinyinfer/models/qwen3.py:219 after the MLP call).
torch::Tensor mlp_forward_mxfp4_residual(torch::Tensor X, torch::Tensor gate, torch::Tensor gate_scale,
                                         torch::Tensor up, torch::Tensor up_scale, torch::Tensor down,
                                         torch::Tensor down_scale, torch::Tensor residual) {
  check_mlp_inputs(X, gate, gate_scale, up, up_scale, down, down_scale);
  TORCH_CHECK(residual.is_cuda() && residual.device() == X.device(), "X/residual device mismatch");
  TORCH_CHECK(residual.sizes() == X.sizes() && residual.scalar_type() == X.scalar_type(),
              "residual must match X's shape and dtype");
  TORCH_CHECK(residual.is_contiguous(), "residual must be contiguous");
  const int64_t N = X.size(0), hidden = X.size(1), inter = gate.size(0);
  const int dtype = X.scalar_type() == at::kHalf ? TI_DTYPE_F16 : TI_DTYPE_BF16;
  c10::DeviceGuard guard(X.device());
  auto O = torch::empty({N, hidden}, X.options());
  auto tmp = torch::empty({N, inter}, X.options());
  const int st = tinyinfer_mlp_forward_mxfp4_residual(
      X.data_ptr(), gate.data_ptr<uint8_t>(), gate_scale.data_ptr<uint8_t>(), up.data_ptr<uint8_t>(),
      up_scale.data_ptr<uint8_t>(), down.data_ptr<uint8_t>(), down_scale.data_ptr<uint8_t>(), (size_t)N,
      (size_t)hidden, (size_t)inter, tmp.data_ptr(), residual.data_ptr(), O.data_ptr(), dtype, TI_PATH_AUTO,
      current_stream());
  check_status(st, "mlp_forward_mxfp4_residual");
  return O;
}

// The decoder layer's MLP half (tinyinfer/models/qwen3.py:210-219):
// X + MLP(RMSNorm(X)), the norm in the MLP's prologue and the residual add in
// its epilogue.  norm_weight is post_attention_layernorm.weight [hidden].
torch::Tensor mlp_forward_mxfp4_rmsnorm(torch::Tensor X, torch::Tensor norm_weight, double eps, torch::Tensor gate,
                                        torch::Tensor gate_scale, torch::Tensor up, torch::Tensor up_scale,
                                        torch::Tensor down, torch::Tensor down_scale) {
  check_mlp_inputs(X, gate, gate_scale, up, up_scale, down, down_scale);
  TORCH_CHECK(norm_weight.is_cuda() && norm_weight.device() == X.device(), "X/norm_weight device mismatch");
  TORCH_CHECK(norm_weight.dim() == 1 && norm_weight.size(0) == X.size(1),
              "norm_weight must have shape [hidden_dim]");
  TORCH_CHECK(norm_weight.scalar_type() == X.scalar_type(), "X/norm_weight dtype mismatch");
  TORCH_CHECK(norm_weight.is_contiguous(), "norm_weight must be contiguous");
  const int64_t N = X.size(0), hidden = X.size(1), inter = gate.size(0);
  const int dtype = X.scalar_type() == at::kHalf ? TI_DTYPE_F16 : TI_DTYPE_BF16;
  c10::DeviceGuard guard(X.device());
  auto O = torch::empty({N, hidden}, X.options());
  auto xn = torch::empty({N, hidden}, X.options());
  auto tmp = torch::empty({N, inter}, X.options());
  const int st = tinyinfer_mlp_forward_mxfp4_rmsnorm(
      X.data_ptr(), norm_weight.data_ptr(), (float)eps, gate.data_ptr<uint8_t>(), gate_scale.data_ptr<uint8_t>(),
      up.data_ptr<uint8_t>(), up_scale.data_ptr<uint8_t>(), down.data_ptr<uint8_t>(), down_scale.data_ptr<uint8_t>(),
      (size_t)N, (size_t)hidden, (size_t)inter, xn.data_ptr(), tmp.data_ptr(), O.data_ptr(), dtype, TI_PATH_AUTO,
      current_stream());
  check_status(st, "mlp_forward_mxfp4_rmsnorm");
  return O;
}

// The reference's rmsnorm_forward (tinyinfer/csrc/bind.cpp:255-293), same
// name, arguments, checks and messages, for fp16 and bf16 (the reference's
// fp32 rows are not built here: they raise).
torch::Tensor rmsnorm_forward(torch::Tensor input, torch::Tensor weight, double eps) {
  TORCH_CHECK(input.is_cuda(), "input must be a CUDA tensor");
  TORCH_CHECK(weight.is_cuda(), "weight must be a CUDA tensor");
  TORCH_CHECK(input.device() == weight.device(), "input/weight must be on the same device");
  TORCH_CHECK(input.dim() >= 1, "input must have at least 1 dimension");
  TORCH_CHECK(weight.dim() == 1, "weight must have shape [D]");
  TORCH_CHECK(input.size(-1) == weight.size(0), "weight size must match input last dimension");
  TORCH_CHECK(input.scalar_type() == weight.scalar_type(), "input/weight dtype mismatch");
  TORCH_CHECK(input.is_contiguous(), "input must be contiguous");
  TORCH_CHECK(weight.is_contiguous(), "weight must be contiguous");
  TORCH_CHECK(input.scalar_type() == at::kHalf || input.scalar_type() == at::kBFloat16,
              "RMSNorm supports fp16 and bf16 only");
  c10::DeviceGuard guard(input.device());
  auto output = torch::empty_like(input);
  const int64_t hidden = input.size(-1);
  const int64_t rows = hidden > 0 ? input.numel() / hidden : 0;
  if (rows == 0) return output;
  const int st = tinyinfer_rmsnorm(input.data_ptr(), weight.data_ptr(), (float)eps, (size_t)rows, (size_t)hidden,
                                   output.data_ptr(), input.scalar_type() == at::kHalf ? TI_DTYPE_F16 : TI_DTYPE_BF16,
                                   current_stream());
  check_status(st, "rmsnorm_forward");
  return output;
}

// X [N, in] @ dequant(W)^T (+ residual) -> [N, out]; W packed [out, in/2], scales [out, in/32].
torch::Tensor mxfp4_linear(torch::Tensor X, torch::Tensor w, torch::Tensor w_scale,
                           c10::optional<torch::Tensor> residual) {
  TORCH_CHECK(X.is_cuda() && w.is_cuda() && w_scale.is_cuda(), "X/w/w_scale must be CUDA tensors");
  TORCH_CHECK(X.device() == w.device() && X.device() == w_scale.device(), "X/w device mismatch");
  TORCH_CHECK(X.dim() == 2 && w.dim() == 2 && w_scale.dim() == 2, "X, w and w_scale must be 2D");
  TORCH_CHECK(X.scalar_type() == at::kHalf || X.scalar_type() == at::kBFloat16,
              "MXFP4 linear only supports FP16 and BF16 activations");
  TORCH_CHECK(w.scalar_type() == at::kByte && w_scale.scalar_type() == at::kByte, "w and w_scale must be uint8");
  const int64_t N = X.size(0), in = X.size(1), out = w.size(0);
  TORCH_CHECK(in % 32 == 0 && out % 32 == 0, "in_features and out_features must be divisible by 32");
  TORCH_CHECK(w.size(1) == in / 2 && w_scale.size(0) == out && w_scale.size(1) == in / 32,
              "w/w_scale shape mismatch");
  TORCH_CHECK(X.is_contiguous() && w.is_contiguous() && w_scale.is_contiguous(), "inputs must be contiguous");
  const void* res = nullptr;
  if (residual.has_value()) {
    const auto& r = residual.value();
    TORCH_CHECK(r.is_cuda() && r.device() == X.device() && r.is_contiguous() && r.dim() == 2 &&
                    r.size(0) == N && r.size(1) == out && r.scalar_type() == X.scalar_type(),
                "residual must be a contiguous [N, out_features] tensor of X's dtype on X's device");
    res = r.data_ptr();
  }
  c10::DeviceGuard guard(X.device());
  auto O = torch::empty({N, out}, X.options());
  const int st = tinyinfer_mxfp4_linear(X.data_ptr(), w.data_ptr<uint8_t>(), w_scale.data_ptr<uint8_t>(),
                                        (size_t)N, (size_t)in, (size_t)out, res, O.data_ptr(),
                                        X.scalar_type() == at::kHalf ? TI_DTYPE_F16 : TI_DTYPE_BF16,
                                        TI_PATH_AUTO, current_stream());
  check_status(st, "mxfp4_linear");
  return O;
}

// packed [rows, K/2] u8 + scale [rows, K/32] u8 -> [rows, K] float32 or bfloat16.
torch::Tensor mxfp4_dequant(torch::Tensor packed, torch::Tensor scale, c10::ScalarType out_dtype) {
  TORCH_CHECK(packed.is_cuda() && scale.is_cuda(), "packed/scale must be CUDA tensors");
  TORCH_CHECK(packed.device() == scale.device(), "packed/scale device mismatch");
  TORCH_CHECK(packed.dim() == 2 && scale.dim() == 2 && packed.size(0) == scale.size(0),
              "packed/scale shape mismatch");
  TORCH_CHECK(packed.scalar_type() == at::kByte && scale.scalar_type() == at::kByte,
              "packed/scale must be uint8");
  TORCH_CHECK(packed.is_contiguous() && scale.is_contiguous(), "packed/scale must be contiguous");
  const int64_t rows = packed.size(0), k = 2 * packed.size(1);
  TORCH_CHECK(k % 32 == 0 && scale.size(1) == k / 32, "scale shape mismatch");
  TORCH_CHECK(out_dtype == at::kFloat || out_dtype == at::kBFloat16, "out_dtype must be float32 or bfloat16");
  c10::DeviceGuard guard(packed.device());
  auto out = torch::empty({rows, k}, packed.options().dtype(out_dtype));
  const int st = tinyinfer_mxfp4_dequant(packed.data_ptr<uint8_t>(), scale.data_ptr<uint8_t>(), (size_t)rows,
                                         (size_t)k, out.data_ptr(),
                                         out_dtype == at::kFloat ? TI_DTYPE_F32 : TI_DTYPE_BF16,
                                         current_stream());
  check_status(st, "mxfp4_dequant");
  return out;
}

// w [rows, K] float32/bfloat16/float16 -> (packed u8 [rows, K/2], scale u8 [rows, K/32], flags i32 [1]).
std::vector<torch::Tensor> mxfp4_quantize(torch::Tensor w) {
  TORCH_CHECK(w.is_cuda(), "w must be a CUDA tensor");
  TORCH_CHECK(w.dim() == 2 && w.size(1) % 32 == 0, "expected [rows,K], K multiple of 32");
  TORCH_CHECK(w.is_contiguous(), "w must be contiguous");
  int dt;
  switch (w.scalar_type()) {
    case at::kFloat: dt = TI_DTYPE_F32; break;
    case at::kBFloat16: dt = TI_DTYPE_BF16; break;
    case at::kHalf: dt = TI_DTYPE_F16; break;
    default: TORCH_CHECK(false, "unsupported weight dtype ", w.scalar_type());
  }
  c10::DeviceGuard guard(w.device());
  const int64_t rows = w.size(0), k = w.size(1);
  auto opts = w.options().dtype(at::kByte);
  auto packed = torch::empty({rows, k / 2}, opts);
  auto scale = torch::empty({rows, k / 32}, opts);
  auto flags = torch::empty({1}, w.options().dtype(at::kInt));
  const int st = tinyinfer_mxfp4_quantize(w.data_ptr(), dt, (size_t)rows, (size_t)k, packed.data_ptr<uint8_t>(),
                                          scale.data_ptr<uint8_t>(),
                                          reinterpret_cast<uint32_t*>(flags.data_ptr<int32_t>()),
                                          current_stream());
  check_status(st, "mxfp4_quantize");
  return {packed, scale, flags};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("mlp_forward_mxfp4", &mlp_forward_mxfp4, "MXFP4 MLP Forward", pybind11::arg("X"),
        pybind11::arg("gate"), pybind11::arg("gate_scale"), pybind11::arg("up"), pybind11::arg("up_scale"),
        pybind11::arg("down"), pybind11::arg("down_scale"));
  m.def("mlp_forward_mxfp4_path", &mlp_forward_mxfp4_path, "MXFP4 MLP Forward with a forced kernel path",
        pybind11::arg("X"), pybind11::arg("gate"), pybind11::arg("gate_scale"), pybind11::arg("up"),
        pybind11::arg("up_scale"), pybind11::arg("down"), pybind11::arg("down_scale"), pybind11::arg("path"));
  m.def("mxfp4_dequant", &mxfp4_dequant, "MXFP4 device dequantization", pybind11::arg("packed"),
        pybind11::arg("scale"), pybind11::arg("out_dtype"));
  m.def("mxfp4_quantize", &mxfp4_quantize, "MXFP4 device quantization", pybind11::arg("w"));
  m.def("mlp_forward_mxfp4_residual", &mlp_forward_mxfp4_residual, "residual + MXFP4 MLP(X)", pybind11::arg("X"),
        pybind11::arg("gate"), pybind11::arg("gate_scale"), pybind11::arg("up"), pybind11::arg("up_scale"),
        pybind11::arg("down"), pybind11::arg("down_scale"), pybind11::arg("residual"));
  m.def("mxfp4_linear", &mxfp4_linear, "MXFP4 linear: X @ dequant(w)^T (+ residual)", pybind11::arg("X"),
        pybind11::arg("w"), pybind11::arg("w_scale"), pybind11::arg("residual") = pybind11::none());
  m.def("mlp_forward_mxfp4_rmsnorm", &mlp_forward_mxfp4_rmsnorm, "X + MXFP4 MLP(RMSNorm(X))", pybind11::arg("X"),
        pybind11::arg("norm_weight"), pybind11::arg("eps"), pybind11::arg("gate"), pybind11::arg("gate_scale"),
        pybind11::arg("up"), pybind11::arg("up_scale"), pybind11::arg("down"), pybind11::arg("down_scale"));
  m.def("rmsnorm_forward", &rmsnorm_forward, "RMSNorm forward", pybind11::arg("input"), pybind11::arg("weight"),
        pybind11::arg("eps"));
  m.attr("PATH_AUTO") = TI_PATH_AUTO;
  m.attr("PATH_SKINNY") = TI_PATH_SKINNY;
  m.attr("PATH_GEMM") = TI_PATH_GEMM;
  m.attr("PATH_DECODE") = TI_PATH_DECODE;
}
