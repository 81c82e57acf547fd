// Zero-padded copies of the projection weights for the padded staged plan
// (head_dim or d_model not a multiple of 8).  The reference pads head_dim inside
// its attention kernel to HD_PAD (torch_transformer_benchmark.py:578, 763-765)
// and masks its GEMM loads; here the library lays the weights out once per call
// in the workspace with each head's rows (or columns) padded from head_dim to a
// multiple of 8 and d_model padded likewise, so that every vectorised kernel of
// the staged plan runs unchanged on 16-byte chunks.  Zero rows give zero q / k /
// v dimensions (zero contribution to q . k, zero context columns) and zero
// columns meet the zero pad of the normalised activations.
#include "common.hpp"
#include "kernels.hpp"

namespace cobra {

namespace {

// i -> (i / gout) * gin + i % gout when i % gout < gin and that is < lim, else -1.
__device__ __forceinline__ int64_t pad_map(int64_t i, int64_t gin, int64_t gout, int64_t lim) {
  const int64_t q = i / gout, rr = i - q * gout;
  if (rr >= gin) return -1;
  const int64_t s = q * gin + rr;
  return s < lim ? s : -1;
}

template <typename T>
__global__ __launch_bounds__(256) void pad_kernel(const T* __restrict__ in, T* __restrict__ out, int64_t in_cols,
                                                  int64_t out_rows, int64_t out_cols, int64_t r_gin, int64_t r_gout,
                                                  int64_t r_lim, int64_t c_gin, int64_t c_gout, int64_t c_lim) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= out_rows * out_cols) return;
  const int64_t r = i / out_cols, c = i - r * out_cols;
  const int64_t sr = pad_map(r, r_gin, r_gout, r_lim), sc = pad_map(c, c_gin, c_gout, c_lim);
  out[i] = (sr >= 0 && sc >= 0) ? in[sr * in_cols + sc] : (T)0;
}

}  // namespace

hipError_t run_pad(const PadArgs& a) {
  if (!a.in || !a.out || a.out_rows < 0 || a.out_cols <= 0 || a.in_cols <= 0) return hipErrorInvalidValue;
  if (a.r_gin <= 0 || a.r_gout <= 0 || a.c_gin <= 0 || a.c_gout <= 0) return hipErrorInvalidValue;
  const int64_t total = a.out_rows * a.out_cols;
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  if (a.elem_bytes == 2)
    hipLaunchKernelGGL((pad_kernel<uint16_t>), dim3((unsigned)blocks), dim3(256), 0, a.stream,
                       static_cast<const uint16_t*>(a.in), static_cast<uint16_t*>(a.out), a.in_cols, a.out_rows,
                       a.out_cols, a.r_gin, a.r_gout, a.r_lim, a.c_gin, a.c_gout, a.c_lim);
  else if (a.elem_bytes == 4)
    hipLaunchKernelGGL((pad_kernel<uint32_t>), dim3((unsigned)blocks), dim3(256), 0, a.stream,
                       static_cast<const uint32_t*>(a.in), static_cast<uint32_t*>(a.out), a.in_cols, a.out_rows,
                       a.out_cols, a.r_gin, a.r_gout, a.r_lim, a.c_gin, a.c_gout, a.c_lim);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace cobra
