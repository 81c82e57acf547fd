// Native steady-state calls of CobraAttentionSublayer.forward (cobra_amd/layer.py) and
// of CobraTransformer.forward in its one-kernel-per-block mode (cobra_amd/model.py).
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

#include <string>
#include <utility>
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
  // attribute was bound (its value must still equal eps).  masked: the launch was bound
  // with a token mask, which every call must then pass ([B, S] bool or uint8 on the
  // device, 0 = padded), and a call without one must not.  on_error(name, code) raises
  // the library's error.
  BoundForward(int64_t handle, const at::Tensor& like, std::vector<at::Tensor> params,
               std::vector<int64_t> snapshot, py::object norm, double eps, bool masked, py::object on_error)
      : handle_(reinterpret_cast<const cobra_layer_launch*>(handle)),
        sizes_(like.sizes().vec()),
        dtype_(like.scalar_type()),
        device_(like.device()),
        params_(std::move(params)),
        snapshot_(std::move(snapshot)),
        norm_(std::move(norm)),
        eps_(eps),
        masked_(masked),
        on_error_(std::move(on_error)) {
    TORCH_CHECK(handle_ != nullptr, "BoundForward: null launch handle");
    TORCH_CHECK(params_.size() == snapshot_.size(), "BoundForward: one snapshot value per parameter");
    TORCH_CHECK(device_.is_cuda(), "BoundForward: the bound input must be a device tensor");
  }

  py::object call(const at::Tensor& x, const c10::optional<at::Tensor>& mask) const {
    if (!x.defined() || x.device() != device_ || x.scalar_type() != dtype_ || x.sizes() != sizes_ ||
        !x.is_contiguous())
      return py::none();
    const uint8_t* m = nullptr;
    if (mask.has_value() != masked_) return py::none();
    if (masked_) {
      const at::Tensor& t = *mask;
      if (!t.defined() || t.device() != device_ || (t.scalar_type() != at::kBool && t.scalar_type() != at::kByte) ||
          t.dim() != 2 || t.size(0) != sizes_[0] || t.size(1) != sizes_[1] || !t.is_contiguous())
        return py::none();
      m = static_cast<const uint8_t*>(t.data_ptr());
    }
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
    const int code = cobra_layer_run(handle_, x.data_ptr(), m, y.data_ptr(), nullptr, s);
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
  bool masked_;
  py::object on_error_;
};

// Steady state of CobraTransformer.forward (cobra_amd/model.py) where every block runs
// as one whole-block kernel: layer 0's norm1 (which also widens x into the fp32
// residual), then one cobra_block_fwd per block, h ping-ponging between two buffers and
// the residual updated in place, the last block writing final_norm's output.  Same
// contract as BoundForward: an input of the bound signature with the parameters and
// epsilon unchanged gets the output; any other call returns None.
class BoundStack {
 public:
  // blocks: per block, in order, w_qkv, b_qkv, w_o, b_o, ln2_w, ln2_b, w1, b1, w2, b2 and
  // the next norm's weight and bias (the next block's norm1, final_norm after the last).
  BoundStack(const at::Tensor& like, std::vector<at::Tensor> params, std::vector<int64_t> snapshot,
             py::object norm, double eps, at::Tensor ln1_w, at::Tensor ln1_b, std::vector<at::Tensor> blocks,
             int64_t heads, int64_t ffn_dim, bool causal, py::object on_error)
      : sizes_(like.sizes().vec()),
        dtype_(like.scalar_type()),
        device_(like.device()),
        params_(std::move(params)),
        snapshot_(std::move(snapshot)),
        norm_(std::move(norm)),
        eps_(eps),
        ln1_w_(std::move(ln1_w)),
        ln1_b_(std::move(ln1_b)),
        blocks_(std::move(blocks)),
        heads_(heads),
        ffn_dim_(ffn_dim),
        causal_(causal),
        on_error_(std::move(on_error)) {
    TORCH_CHECK(params_.size() == snapshot_.size(), "BoundStack: one snapshot value per parameter");
    TORCH_CHECK(device_.is_cuda() && sizes_.size() == 3, "BoundStack: the bound input must be a [B, S, D] device tensor");
    TORCH_CHECK(dtype_ == at::kHalf || dtype_ == at::kFloat, "BoundStack: fp16 or fp32 activations");
    TORCH_CHECK(!blocks_.empty() && blocks_.size() % kPerBlock == 0, "BoundStack: 12 tensors per block");
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
    const int64_t B = sizes_[0], S = sizes_[1], D = sizes_[2], T = B * S;
    const int xdt = dtype_ == at::kHalf ? COBRA_F16 : COBRA_F32;
    const float eps = static_cast<float>(eps_);
    const size_t n = blocks_.size() / kPerBlock;
    at::Tensor r = at::detail::empty_cuda({T, D}, at::kFloat, device_, c10::nullopt);
    at::Tensor h = at::detail::empty_cuda({T, D}, at::kHalf, device_, c10::nullopt);
    at::Tensor hn = n > 1 ? at::detail::empty_cuda({T, D}, at::kHalf, device_, c10::nullopt) : at::Tensor();
    at::Tensor out = at::detail::empty_cuda(sizes_, dtype_, device_, c10::nullopt);
    const hipStream_t s = c10::hip::getCurrentHIPStream(device_.index()).stream();
    check("cobra_ln_fwd", cobra_ln_fwd(x.data_ptr(), xdt, nullptr, 0, ln1_w_.data_ptr<float>(),
                                       ln1_b_.data_ptr<float>(), nullptr, 0, r.data_ptr<float>(), h.data_ptr(),
                                       COBRA_F16, T, D, eps, s));
    for (size_t i = 0; i < n; ++i) {
      const at::Tensor* b = &blocks_[kPerBlock * i];
      const bool last = i + 1 == n;
      void* o = last ? out.data_ptr() : hn.data_ptr();
      check("cobra_block_fwd",
            cobra_block_fwd(h.data_ptr(), r.data_ptr<float>(), nullptr, b[0].data_ptr(), b[1].data_ptr<float>(),
                            b[2].data_ptr(), b[3].data_ptr<float>(), b[4].data_ptr<float>(), b[5].data_ptr<float>(),
                            b[6].data_ptr(), b[7].data_ptr<float>(), b[8].data_ptr(), b[9].data_ptr<float>(),
                            b[10].data_ptr<float>(), b[11].data_ptr<float>(), r.data_ptr<float>(), o,
                            last ? xdt : COBRA_F16, 0, B, S, D, heads_, ffn_dim_, causal_ ? 1 : 0, eps, s));
      if (!last) std::swap(h, hn);
    }
    return py::cast(std::move(out));
  }

 private:
  static constexpr size_t kPerBlock = 12;

  void check(const char* fn, int code) const {
    if (code != 0) {
      on_error_(fn, code);  // raises
      throw std::runtime_error(std::string(fn) + " failed");
    }
  }

  std::vector<int64_t> sizes_;
  at::ScalarType dtype_;
  at::Device device_;
  std::vector<at::Tensor> params_;
  std::vector<int64_t> snapshot_;
  py::object norm_;
  double eps_;
  at::Tensor ln1_w_, ln1_b_;
  std::vector<at::Tensor> blocks_;
  int64_t heads_, ffn_dim_;
  bool causal_;
  py::object on_error_;
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Native steady-state forward of the cobra_amd attention sublayer";
  py::class_<BoundForward>(m, "BoundForward")
      .def(py::init<int64_t, const at::Tensor&, std::vector<at::Tensor>, std::vector<int64_t>, py::object, double,
                    bool, py::object>())
      .def("__call__", &BoundForward::call, py::arg("x"), py::arg("mask") = py::none());
  py::class_<BoundStack>(m, "BoundStack")
      .def(py::init<const at::Tensor&, std::vector<at::Tensor>, std::vector<int64_t>, py::object, double, at::Tensor,
                    at::Tensor, std::vector<at::Tensor>, int64_t, int64_t, bool, py::object>())
      .def("__call__", &BoundStack::call);
}
