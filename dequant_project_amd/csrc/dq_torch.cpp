// PyTorch-ROCm extension `dequant_cuda`: the reference's Python surface
// (kernels/bindings.cpp:5-17, prototypes kernels/dequant_cuda.h:10-20) over the
// C ABI of include/dequant_hip.h. This layer only turns tensors into operand
// descriptors, allocates outputs (as the reference's launchers do with
// torch::empty) and picks the current HIP stream; validation and launches
// live behind the C ABI. Errors raise RuntimeError with the reference's text.

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "dequant_hip.h"

namespace {

dq_tensor describe(const at::Tensor& t) {
  dq_tensor d{};
  d.data = t.data_ptr();
  d.is_device = t.is_cuda() ? 1 : 0;
  d.device = t.is_cuda() ? t.get_device() : -1;
  switch (t.scalar_type()) {
    case at::kInt: d.dtype = DQ_DTYPE_INT32; break;
    case at::kHalf: d.dtype = DQ_DTYPE_FLOAT16; break;
    case at::kFloat: d.dtype = DQ_DTYPE_FLOAT32; break;
    default: d.dtype = DQ_DTYPE_OTHER; break;
  }
  d.contiguous = t.is_contiguous() ? 1 : 0;
  d.ndim = static_cast<int32_t>(t.dim());
  for (int i = 0; i < d.ndim && i < 4; ++i) d.sizes[i] = t.size(i);
  return d;
}

void raise_if(int status) {
  if (status != DQ_OK) throw std::runtime_error(dq_last_error());
}

dq_stream_t current_stream(const at::Tensor& t) {
  return reinterpret_cast<dq_stream_t>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

const uint16_t* half_ptr(const at::Tensor& t) { return reinterpret_cast<const uint16_t*>(t.data_ptr()); }

}  // namespace

// kernels/smoke.cu:15-25
torch::Tensor add_one(torch::Tensor x) {
  if (!x.is_cuda()) throw std::runtime_error("x must be a CUDA tensor");
  if (x.scalar_type() != at::kFloat) throw std::runtime_error("x must be float32");
  auto xc = x.contiguous();
  const c10::DeviceGuard guard(x.device());
  auto out = torch::empty_like(xc);
  raise_if(dq_add_one(xc.data_ptr<float>(), out.data_ptr<float>(), xc.numel(), current_stream(xc)));
  return out;
}

// kernels/dequant_gemv.cu:339-386
torch::Tensor gemv(torch::Tensor x, torch::Tensor qweight, torch::Tensor scales,
                   std::optional<torch::Tensor> zeros, int64_t bits, int64_t group_size, bool symmetric,
                   bool interleaved) {
  const dq_tensor dx = describe(x), dw = describe(qweight), ds = describe(scales);
  dq_tensor dz{};
  if (zeros) dz = describe(*zeros);
  raise_if(dq_check_gemv(&dx, &dw, &ds, zeros ? &dz : nullptr, bits, group_size, symmetric));

  const c10::DeviceGuard guard(x.device());
  const int64_t M = x.size(0), K = x.size(1), N = qweight.size(0);
  auto y = torch::empty({M, N}, x.options());
  raise_if(dq_gemv(half_ptr(x), reinterpret_cast<const uint32_t*>(qweight.data_ptr()), half_ptr(scales),
                   zeros ? half_ptr(*zeros) : nullptr, reinterpret_cast<uint16_t*>(y.data_ptr()), M, N, K, bits,
                   group_size, symmetric, interleaved, current_stream(x)));
  return y;
}

// Grouped launch of several GEMVs of one format and one M (no reference
// counterpart; see dq_gemv_batched). Each problem is validated exactly as
// gemv() validates its arguments.
std::vector<torch::Tensor> gemv_batched(std::vector<torch::Tensor> xs, std::vector<torch::Tensor> qweights,
                                        std::vector<torch::Tensor> scales,
                                        std::vector<std::optional<torch::Tensor>> zeros, int64_t bits,
                                        std::vector<int64_t> group_sizes, bool symmetric, bool interleaved) {
  const size_t n = xs.size();
  if (n == 0 || n > DQ_MAX_BATCH)
    throw std::runtime_error("gemv_batched takes 1.." + std::to_string(DQ_MAX_BATCH) + " problems");
  if (qweights.size() != n || scales.size() != n || zeros.size() != n || group_sizes.size() != n)
    throw std::runtime_error("gemv_batched: xs, qweights, scales, zeros and group_sizes differ in length");
  std::vector<dq_gemv_problem> probs(n);
  std::vector<torch::Tensor> ys;
  ys.reserve(n);
  for (size_t i = 0; i < n; ++i) {
    const dq_tensor dx = describe(xs[i]), dw = describe(qweights[i]), ds = describe(scales[i]);
    dq_tensor dz{};
    if (zeros[i]) dz = describe(*zeros[i]);
    if (dq_check_gemv(&dx, &dw, &ds, zeros[i] ? &dz : nullptr, bits, group_sizes[i], symmetric) != DQ_OK)
      throw std::runtime_error("problem " + std::to_string(i) + ": " + dq_last_error());
    if (xs[i].size(0) != xs[0].size(0)) throw std::runtime_error("gemv_batched: all problems must share M");
    if (xs[i].device() != xs[0].device()) throw std::runtime_error("gemv_batched: all problems must share a device");
    ys.push_back(torch::empty({xs[i].size(0), qweights[i].size(0)}, xs[i].options()));
    probs[i] = dq_gemv_problem{half_ptr(xs[i]), reinterpret_cast<const uint32_t*>(qweights[i].data_ptr()),
                               half_ptr(scales[i]), zeros[i] ? half_ptr(*zeros[i]) : nullptr,
                               reinterpret_cast<uint16_t*>(ys[i].data_ptr()), qweights[i].size(0),
                               xs[i].size(1), group_sizes[i]};
  }
  const c10::DeviceGuard guard(xs[0].device());
  raise_if(dq_gemv_batched(probs.data(), static_cast<int>(n), xs[0].size(0), bits, symmetric, interleaved,
                           current_stream(xs[0])));
  return ys;
}

// Grouped GEMV with a fused activation prologue (no reference counterpart; see
// dq_gemv_prologue_batched): prologue 1 = RMSNorm (auxs[i] = gamma, fp16 [K]),
// 2 = SwiGLU (xs[i] = gate output, auxs[i] = up output, both fp16 [M, K]).
std::vector<torch::Tensor> gemv_prologue(std::vector<torch::Tensor> xs, std::vector<torch::Tensor> auxs,
                                         int64_t prologue, double eps, std::vector<torch::Tensor> qweights,
                                         std::vector<torch::Tensor> scales,
                                         std::vector<std::optional<torch::Tensor>> zeros, int64_t bits,
                                         std::vector<int64_t> group_sizes, bool symmetric, bool interleaved) {
  const size_t n = xs.size();
  if (n == 0 || n > DQ_MAX_BATCH)
    throw std::runtime_error("gemv_prologue takes 1.." + std::to_string(DQ_MAX_BATCH) + " problems");
  if (auxs.size() != n || qweights.size() != n || scales.size() != n || zeros.size() != n ||
      group_sizes.size() != n)
    throw std::runtime_error("gemv_prologue: xs, auxs, qweights, scales, zeros and group_sizes differ in length");
  std::vector<dq_gemv_problem> probs(n);
  std::vector<const void*> aux_ptrs(n);
  std::vector<torch::Tensor> ys;
  ys.reserve(n);
  for (size_t i = 0; i < n; ++i) {
    const dq_tensor dx = describe(xs[i]), dw = describe(qweights[i]), ds = describe(scales[i]);
    dq_tensor dz{};
    if (zeros[i]) dz = describe(*zeros[i]);
    if (dq_check_gemv(&dx, &dw, &ds, zeros[i] ? &dz : nullptr, bits, group_sizes[i], symmetric) != DQ_OK)
      throw std::runtime_error("problem " + std::to_string(i) + ": " + dq_last_error());
    if (xs[i].size(0) != xs[0].size(0)) throw std::runtime_error("gemv_prologue: all problems must share M");
    if (xs[i].device() != xs[0].device()) throw std::runtime_error("gemv_prologue: all problems must share a device");
    const torch::Tensor& a = auxs[i];
    const bool shape_ok = prologue == DQ_PROLOGUE_SWIGLU ? a.sizes() == xs[i].sizes()
                                                         : (a.dim() == 1 && a.size(0) == xs[i].size(1));
    if (a.scalar_type() != at::kHalf || !a.is_contiguous() || a.device() != xs[i].device() || !shape_ok)
      throw std::runtime_error("problem " + std::to_string(i) + ": aux must be a contiguous float16 tensor on " +
                               "x's device, " + (prologue == DQ_PROLOGUE_SWIGLU ? "shaped like x" : "of shape [K]"));
    aux_ptrs[i] = a.data_ptr();
    ys.push_back(torch::empty({xs[i].size(0), qweights[i].size(0)}, xs[i].options()));
    probs[i] = dq_gemv_problem{half_ptr(xs[i]), reinterpret_cast<const uint32_t*>(qweights[i].data_ptr()),
                               half_ptr(scales[i]), zeros[i] ? half_ptr(*zeros[i]) : nullptr,
                               reinterpret_cast<uint16_t*>(ys[i].data_ptr()), qweights[i].size(0),
                               xs[i].size(1), group_sizes[i]};
  }
  const c10::DeviceGuard guard(xs[0].device());
  raise_if(dq_gemv_prologue_batched(probs.data(), aux_ptrs.data(), static_cast<int>(n), xs[0].size(0), bits,
                                    symmetric, interleaved, static_cast<int>(prologue), static_cast<float>(eps),
                                    current_stream(xs[0])));
  return ys;
}

// Fused small GEMM for 1 <= M <= DQ_MAX_GEMM_M (no reference counterpart; see
// dq_gemm_small): the product the reference's M > 8 path (dequantize, then
// F.linear over the fp16 weight) computes, in one pass over the packed bytes.
torch::Tensor gemm_small(torch::Tensor x, torch::Tensor qweight, torch::Tensor scales,
                         std::optional<torch::Tensor> zeros, int64_t bits, int64_t group_size, bool symmetric,
                         bool interleaved) {
  const dq_tensor dx = describe(x), dw = describe(qweight), ds = describe(scales);
  dq_tensor dz{};
  if (zeros) dz = describe(*zeros);
  raise_if(dq_check_gemm_small(&dx, &dw, &ds, zeros ? &dz : nullptr, bits, group_size, symmetric));

  const c10::DeviceGuard guard(x.device());
  const int64_t M = x.size(0), K = x.size(1), N = qweight.size(0);
  auto y = torch::empty({M, N}, x.options());
  const dq_gemv_problem prob{half_ptr(x), reinterpret_cast<const uint32_t*>(qweight.data_ptr()), half_ptr(scales),
                             zeros ? half_ptr(*zeros) : nullptr, reinterpret_cast<uint16_t*>(y.data_ptr()), N, K,
                             group_size};
  raise_if(dq_gemm_small(&prob, 1, M, bits, symmetric, interleaved, current_stream(x)));
  return y;
}

// kernels/dequant_gemv.cu:310-337
torch::Tensor dequantize(torch::Tensor qweight, torch::Tensor scales, std::optional<torch::Tensor> zeros,
                         int64_t bits, int64_t group_size, bool symmetric, bool interleaved, int64_t K) {
  const dq_tensor dw = describe(qweight), ds = describe(scales);
  dq_tensor dz{};
  if (zeros) dz = describe(*zeros);
  raise_if(dq_check_dequantize(&dw, &ds, zeros ? &dz : nullptr, bits, group_size, symmetric, K));

  const c10::DeviceGuard guard(qweight.device());
  const int64_t N = qweight.size(0);
  auto out = torch::empty({N, K}, scales.options());
  raise_if(dq_dequantize(reinterpret_cast<const uint32_t*>(qweight.data_ptr()), half_ptr(scales),
                         zeros ? half_ptr(*zeros) : nullptr, reinterpret_cast<uint16_t*>(out.data_ptr()), N, K,
                         bits, group_size, symmetric, interleaved, current_stream(qweight)));
  return out;
}

// No reference counterpart: the codes themselves, for the bit-exact unpack check
// against dequant/packer.py:164-174.
torch::Tensor unpack(torch::Tensor qweight, int64_t bits, bool interleaved, int64_t K) {
  const dq_tensor dw = describe(qweight);
  raise_if(dq_check_unpack(&dw, bits, K));
  const c10::DeviceGuard guard(qweight.device());
  const int64_t N = qweight.size(0);
  auto out = torch::empty({N, K}, qweight.options().dtype(at::kInt));
  raise_if(dq_unpack(reinterpret_cast<const uint32_t*>(qweight.data_ptr()), out.data_ptr<int32_t>(), N, K,
                     bits, interleaved, current_stream(qweight)));
  return out;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("add_one", &add_one, "add one (HIP, gfx950)", py::arg("x"));
  m.def("gemv", &gemv, "packed-weight GEMV, fp16 [M,K] x [N,K]^T -> [M,N]", py::arg("x"), py::arg("qweight"),
        py::arg("scales"), py::arg("zeros"), py::arg("bits"), py::arg("group_size"), py::arg("symmetric"),
        py::arg("interleaved"));
  m.def("gemv_batched", &gemv_batched, "grouped packed-weight GEMVs of one format in one launch",
        py::arg("xs"), py::arg("qweights"), py::arg("scales"), py::arg("zeros"), py::arg("bits"),
        py::arg("group_sizes"), py::arg("symmetric"), py::arg("interleaved"));
  m.def("gemv_prologue", &gemv_prologue,
        "grouped packed-weight GEMVs (M = 1) with a fused RMSNorm (1) or SwiGLU (2) activation prologue",
        py::arg("xs"), py::arg("auxs"), py::arg("prologue"), py::arg("eps"), py::arg("qweights"), py::arg("scales"),
        py::arg("zeros"), py::arg("bits"), py::arg("group_sizes"), py::arg("symmetric"), py::arg("interleaved"));
  m.def("gemm_small", &gemm_small, "packed-weight GEMM for 1 <= M <= 64: x @ dequantize(W)^T in one pass",
        py::arg("x"), py::arg("qweight"), py::arg("scales"), py::arg("zeros"), py::arg("bits"),
        py::arg("group_size"), py::arg("symmetric"), py::arg("interleaved"));
  m.def("dequantize", &dequantize, "materialize a packed weight as fp16 [N,K]", py::arg("qweight"),
        py::arg("scales"), py::arg("zeros"), py::arg("bits"), py::arg("group_size"), py::arg("symmetric"),
        py::arg("interleaved"), py::arg("K"));
  m.def("unpack", &unpack, "packed words -> int32 codes [N,K] in logical order", py::arg("qweight"),
        py::arg("bits"), py::arg("interleaved"), py::arg("K"));
  m.attr("library_version") = dq_version();
}
