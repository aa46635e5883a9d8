// Host-side descriptor builder of the AdamW path (_pm_host, a CPython
// extension compiled against torch's headers; no GPU call, no device code).
//
// torch's fused Adam is handed a param group's tensors as Python lists
// (torch/optim/adam.py:803-898). Reading
// each tensor's pointer, size and dtype from Python costs a method call per
// attribute and tensor, most of the host time of a step over a few hundred
// tensors; fill_adam reads them in one C++ pass and writes the pm_adam_tensor
// array that pm_adam_step (include/panmuon.h) takes, checking on the way what
// that entry point needs of the lists.
#include <torch/extension.h>

#include <cstdint>
#include <vector>

#include "../../include/panmuon.h"

namespace {

int32_t dtype_code(c10::ScalarType s) {
  switch (s) {
    case c10::ScalarType::Float: return PM_DTYPE_F32;
    case c10::ScalarType::BFloat16: return PM_DTYPE_BF16;
    case c10::ScalarType::Half: return PM_DTYPE_F16;
    default: return -1;
  }
}

// Status of fill_adam.
enum FillStatus : int { kFilled = 0, kGeneral = 1 };

// Fills the n-entry pm_adam_tensor array at address `out` from the lists of
// one fused-Adam call (max_exp_avg_sqs empty without amsgrad). Returns
// kFilled when every tensor is on params[0]'s HIP device with a dtype
// pm_adam_step takes (max_exp_avg_sq of exp_avg_sq's dtype, steps float32),
// and every param, grad and state tensor is contiguous with its param's
// element count: pm_adam_step walks the five as flat arrays of one length,
// which is right only when their memory orders agree. kGeneral otherwise
// (the caller's general path splits the lists); the array is complete only
// on kFilled. List lengths that differ raise. hip_only = false also fills
// from CPU tensors, for the CPU tests of the array's layout (pm_adam_step
// needs device pointers: the product path keeps the default).
int fill_adam(int64_t out, const std::vector<at::Tensor>& params, const std::vector<at::Tensor>& grads,
              const std::vector<at::Tensor>& exp_avgs, const std::vector<at::Tensor>& exp_avg_sqs,
              const std::vector<at::Tensor>& max_exp_avg_sqs, const std::vector<at::Tensor>& steps,
              bool hip_only) {
  const size_t n = params.size();
  TORCH_CHECK(grads.size() == n && exp_avgs.size() == n && exp_avg_sqs.size() == n && steps.size() == n,
              "fill_adam: the tensor lists differ in length");
  const bool amsgrad = !max_exp_avg_sqs.empty();
  TORCH_CHECK(!amsgrad || max_exp_avg_sqs.size() == n, "fill_adam: max_exp_avg_sqs differs in length");
  if (n == 0) return kFilled;
  TORCH_CHECK(out != 0, "fill_adam: null descriptor array");
  auto* d = reinterpret_cast<pm_adam_tensor*>(out);
  const c10::Device dev = params[0].device();
  if (hip_only && !dev.is_cuda()) return kGeneral;
  for (size_t i = 0; i < n; ++i) {
    const at::Tensor& p = params[i];
    const at::Tensor& g = grads[i];
    const at::Tensor& m = exp_avgs[i];
    const at::Tensor& v = exp_avg_sqs[i];
    const at::Tensor& s = steps[i];
    if (p.device() != dev || g.device() != dev || m.device() != dev || v.device() != dev || s.device() != dev)
      return kGeneral;
    const int64_t numel = p.numel();
    if (!p.is_contiguous() || !g.is_contiguous() || !m.is_contiguous() || !v.is_contiguous() ||
        g.numel() != numel || m.numel() != numel || v.numel() != numel || s.numel() != 1)
      return kGeneral;
    const int32_t cp = dtype_code(p.scalar_type()), cg = dtype_code(g.scalar_type());
    const int32_t cm = dtype_code(m.scalar_type()), cv = dtype_code(v.scalar_type());
    if (cp < 0 || cg < 0 || cm < 0 || cv < 0 || s.scalar_type() != c10::ScalarType::Float) return kGeneral;
    void* x = nullptr;
    if (amsgrad) {
      const at::Tensor& t = max_exp_avg_sqs[i];
      if (t.device() != dev || t.scalar_type() != v.scalar_type() || !t.is_contiguous() || t.numel() != numel)
        return kGeneral;
      x = t.data_ptr();
    }
    pm_adam_tensor& e = d[i];
    e.param = p.data_ptr();
    e.grad = g.data_ptr();
    e.exp_avg = m.data_ptr();
    e.exp_avg_sq = v.data_ptr();
    e.max_exp_avg_sq = x;
    e.step = static_cast<float*>(s.data_ptr());
    e.numel = numel;
    e.param_dtype = cp;
    e.grad_dtype = cg;
    e.exp_avg_dtype = cm;
    e.exp_avg_sq_dtype = cv;
  }
  return kFilled;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "pan2_amd host helpers: pm_adam_tensor descriptors from torch tensor lists";
  m.def("fill_adam", &fill_adam, "Fill a pm_adam_tensor array from fused-Adam tensor lists", pybind11::arg("out"),
        pybind11::arg("params"), pybind11::arg("grads"), pybind11::arg("exp_avgs"), pybind11::arg("exp_avg_sqs"),
        pybind11::arg("max_exp_avg_sqs"), pybind11::arg("steps"), pybind11::arg("hip_only") = true);
  m.attr("FILLED") = static_cast<int>(kFilled);
  m.attr("GENERAL") = static_cast<int>(kGeneral);
  m.attr("DESC_BYTES") = static_cast<int>(sizeof(pm_adam_tensor));
}
