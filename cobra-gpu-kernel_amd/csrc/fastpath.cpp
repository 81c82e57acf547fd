// Native steady-state call of CobraAttentionSublayer.forward (cobra_amd/layer.py).
//
// At the small shapes one sublayer forward is a single ~7 us kernel, and the Python
// around its launch (signature and parameter-version checks, the output allocation,
// the ctypes call) took about as long as the kernel, so back-to-back forwards were
// bound by the host.  BoundForward holds one bound launch (cobra_layer_bind) and does
// those steps in C++: for an input of the bound signature, with the module's
// parameters and LayerNorm epsilon unchanged since the bind, it allocates y with the
// caching allocator, launches on the device's current stream and returns y; for any
// other call it returns None and the module takes its general path.  It never
// computes anything itself: the launch is the library's (libcobra_amd.so).
#include <torch/extension.h>

#include <ATen/hip/EmptyTensor.h>
#include <c10/hip/HIPStream.h>

#include <vector>

#include "cobra_amd.h"

namespace {

class BoundForward {
 public:
  // handle: a cobra_layer_launch* from cobra_layer_bind (owned by the caller, which
  // keeps it and every buffer it names alive as long as this object).  like: an input
  // of the bound signature.  params / snapshot: the tensors the bound weights were
  // packed from, and for each its version counter (or, for an inference tensor, which
  // keeps none, its data pointer) at packing time.  norm: the module whose `eps`
  // attribute was bound (its value must still equal eps).  on_error(name, code) raises
  // the library's error.
  BoundForward(int64_t handle, const at::Tensor& like, std::vector<at::Tensor> params,
               std::vector<int64_t> snapshot, py::object norm, double eps, py::object on_error)
      : handle_(reinterpret_cast<const cobra_layer_launch*>(handle)),
        sizes_(like.sizes().vec()),
        dtype_(like.scalar_type()),
        device_(like.device()),
        params_(std::move(params)),
        snapshot_(std::move(snapshot)),
        norm_(std::move(norm)),
        eps_(eps),
        on_error_(std::move(on_error)) {
    TORCH_CHECK(handle_ != nullptr, "BoundForward: null launch handle");
    TORCH_CHECK(params_.size() == snapshot_.size(), "BoundForward: one snapshot value per parameter");
    TORCH_CHECK(device_.is_cuda(), "BoundForward: the bound input must be a device tensor");
  }

  py::object call(const at::Tensor& x) const {
    if (!x.defined() || x.device() != device_ || x.scalar_type() != dtype_ || x.sizes() != sizes_ ||
        !x.is_contiguous())
      return py::none();
    for (size_t i = 0; i < params_.size(); ++i) {
      const at::Tensor& p = params_[i];
      const int64_t now = p.is_inference() ? reinterpret_cast<int64_t>(p.data_ptr()) : p._version();
      if (now != snapshot_[i]) return py::none();
    }
    if (norm_.attr("eps").cast<double>() != eps_) return py::none();
    // The device allocator directly (the caching allocator, as empty_like reaches it
    // after two dispatcher round trips); x is contiguous, so y has x's layout.
    at::Tensor y = at::detail::empty_cuda(sizes_, dtype_, device_, c10::nullopt);
    const hipStream_t s = c10::hip::getCurrentHIPStream(device_.index()).stream();
    const int code = cobra_layer_run(handle_, x.data_ptr(), nullptr, y.data_ptr(), nullptr, s);
    if (code != 0) {
      on_error_("cobra_layer_run", code);  // raises
      throw std::runtime_error("cobra_layer_run failed");
    }
    return py::cast(std::move(y));
  }

 private:
  const cobra_layer_launch* handle_;
  std::vector<int64_t> sizes_;
  at::ScalarType dtype_;
  at::Device device_;
  std::vector<at::Tensor> params_;
  std::vector<int64_t> snapshot_;
  py::object norm_;
  double eps_;
  py::object on_error_;
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Native steady-state forward of the cobra_amd attention sublayer";
  py::class_<BoundForward>(m, "BoundForward")
      .def(py::init<int64_t, const at::Tensor&, std::vector<at::Tensor>, std::vector<int64_t>, py::object, double,
                    py::object>())
      .def("__call__", &BoundForward::call);
}
