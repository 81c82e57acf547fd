// Row LayerNorm with optional residual branch and row mask:
//   r = (x (+ branch)) (* m);  y = LN(r) (* m)
//
// Replaces the reference's _add_ln_kernel / _tl_add_ln
// (torch_transformer_benchmark.py:491-569): two-pass fp32 statistics over the
// row held in registers (mean, then centred biased variance, /N), eps inside
// the square root, affine, cast on store.  The row mask m (0 for a padded row,
// 1 otherwise) multiplies the residual (MASK_RESID) and/or the output
// (MASK_OUT) as the reference kernel does (TTB:511-534).  A null gamma (and beta)
// means a LayerNorm without elementwise affine.  x and y are fp16, fp32 or bf16
// each; the branch fp16 or fp32.
//
// Layout: LPR lanes own one row, each lane holds NCH chunks of 8 consecutive
// elements (16 B of fp16 or bf16, 32 B of fp32), so every global access is a full
// vector access and the row reductions never leave the LPR-lane group.
#include "common.hpp"
#include "kernels.hpp"

namespace cobra {

// Rows up to 1024 wide: eight waves per SIMD (<= 64 VGPRs), so that 8192 rows
// of 1024 -- one row per wave -- are all in flight at once on 256 CUs instead
// of in two rounds.  Wider rows hold more registers and keep the default.
template <typename TX, typename TY, int LPR, int NCH>
__global__ __launch_bounds__(256, NCH <= 2 ? 8 : 1) void ln_rows_kernel(const TX* __restrict__ x, const void* __restrict__ branch,
                                                      int branch_f32, const float* __restrict__ gamma,
                                                      const float* __restrict__ beta, float* __restrict__ resid_out,
                                                      TY* __restrict__ y, int64_t rows, int d, float eps,
                                                      const uint8_t* __restrict__ row_mask, int mask_resid,
                                                      int mask_out) {
  constexpr int RPW = 64 / LPR;  // rows per wave
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane % LPR;
  const int64_t row = ((int64_t)blockIdx.x * (blockDim.x >> 6) + wave) * RPW + lane / LPR;
  const bool active = row < rows;
  const int nch = d >> 3;
  const int64_t base = row * d;
  const float mv = (row_mask && active) ? (row_mask[row] != 0 ? 1.f : 0.f) : 1.f;

  float v[NCH][8];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int ch = li + c * LPR;
    if (active && ch < nch) {
      load8(x + base + ch * 8, v[c]);
      if (branch) {
        float bv[8];
        if (branch_f32)
          load8(static_cast<const float*>(branch) + base + ch * 8, bv);
        else
          load8(static_cast<const f16*>(branch) + base + ch * 8, bv);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] += bv[i];
      }
      if (mask_resid) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[c][i] *= mv;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[c][i];
  }
  const float mean = group_sum<LPR>(s) / (float)d;

  float q = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (active && li + c * LPR < nch) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float t = v[c][i] - mean;
        q += t * t;
      }
    }
  }
  const float rstd = rsqrtf(group_sum<LPR>(q) / (float)d + eps);

#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int ch = li + c * LPR;
    if (!(active && ch < nch)) continue;
    if (resid_out) store8(resid_out + base + ch * 8, v[c]);
    float o[8];
    if (gamma) {
      const f32x4 g0 = *reinterpret_cast<const f32x4*>(gamma + ch * 8);
      const f32x4 g1 = *reinterpret_cast<const f32x4*>(gamma + ch * 8 + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(beta + ch * 8);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(beta + ch * 8 + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = (v[c][i] - mean) * rstd * g0[i] + b0[i];
        o[i + 4] = (v[c][i + 4] - mean) * rstd * g1[i] + b1[i];
      }
    } else {  // no elementwise affine
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (v[c][i] - mean) * rstd;
    }
    if (mask_out) {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] *= mv;
    }
    store8(y + base + ch * 8, o);
  }
}

// Plain rows of 512 * NCH (the staged sublayer's LN1 and LN2 passes at d_model 512 /
// 1024): no branch, mask or residual store, the width fixed at compile time, one row
// per wave.  Without the generic kernel's option handling (branches and address
// arithmetic around every chunk) the pass runs ~0.8 us faster at 8192 x 1024.
// BR: r = x + branch (fp16 branch, the sum in fp32) is normalised instead of x.
template <typename TX, typename TY, int NCH, bool BR>
__global__ __launch_bounds__(256) void ln_plain_kernel(const TX* __restrict__ x, const f16* __restrict__ branch,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, TY* __restrict__ y,
                                                       int64_t rows, float eps) {
  constexpr int D = 512 * NCH;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // wave-uniform; no barrier follows
  float gv[NCH][8], bv[NCH][8];
  if (gamma) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      load8(gamma + 512 * c + 8 * lane, gv[c]);
      load8(beta + 512 * c + 8 * lane, bv[c]);
    }
  }
  float v[NCH][8];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) load8(x + r * D + 512 * c + 8 * lane, v[c]);
  if constexpr (BR) {
    float bb[NCH][8];
#pragma unroll
    for (int c = 0; c < NCH; ++c) load8(branch + r * D + 512 * c + 8 * lane, bb[c]);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] += bb[c][i];
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[c][i];
  const float mean = group_sum<64>(s) * (1.0f / D);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float t = v[c][i] - mean;
      q += t * t;
    }
  const float rstd = rsqrtf(group_sum<64>(q) * (1.0f / D) + eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = gamma ? (v[c][i] - mean) * rstd * gv[c][i] + bv[c][i] : (v[c][i] - mean) * rstd;
    store8(y + r * D + 512 * c + 8 * lane, o);
  }
}

// Any width, any row strides (element-wise, one wave per row, lane l holding
// columns l, l + 64, ...): rows not a multiple of 8 wide, or rows inside wider
// buffers, such as the padded staged plan's LN1 (x [T, D] -> h [T, Dp] with the
// pad columns zeroed) and LN2 (x [T, D] + branch [T, Dp]).  Same arithmetic as
// ln_rows_kernel: two-pass fp32 statistics, eps inside the square root.
template <typename TX, typename TY, int NE>
__global__ __launch_bounds__(256) void ln_any_kernel(const TX* __restrict__ x, int64_t ldx, const void* __restrict__ branch,
                                                     int branch_f32, int64_t ldb, const float* __restrict__ gamma,
                                                     const float* __restrict__ beta, float* __restrict__ resid_out,
                                                     int64_t ldr, TY* __restrict__ y, int64_t ldy, int64_t rows, int d,
                                                     float eps, const uint8_t* __restrict__ row_mask, int mask_resid,
                                                     int mask_out) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // wave-uniform; no barrier follows
  const float mv = row_mask ? (row_mask[r] != 0 ? 1.f : 0.f) : 1.f;
  float v[NE];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int c = lane + 64 * k;
    v[k] = 0.f;
    if (c < d) {
      v[k] = (float)x[r * ldx + c];
      if (branch)
        v[k] += branch_f32 ? static_cast<const float*>(branch)[r * ldb + c]
                           : (float)static_cast<const f16*>(branch)[r * ldb + c];
      if (mask_resid) v[k] *= mv;
    }
    s += v[k];
  }
  const float mean = group_sum<64>(s) / (float)d;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < NE; ++k)
    if (lane + 64 * k < d) {
      const float t = v[k] - mean;
      q += t * t;
    }
  const float rstd = rsqrtf(group_sum<64>(q) / (float)d + eps);
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int c = lane + 64 * k;
    if (c < d) {
      if (resid_out) resid_out[r * ldr + c] = v[k];
      float o = (v[k] - mean) * rstd;
      if (gamma) o = o * gamma[c] + beta[c];
      if (mask_out) o *= mv;
      y[r * ldy + c] = (TY)o;
    } else if (c < ldy) {
      y[r * ldy + c] = (TY)0.0f;
    }
  }
}

template <typename TX, typename TY, int NE>
static hipError_t launch_ln_any(const LnArgs& a) {
  const int64_t blocks = (a.rows + 3) / 4;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((ln_any_kernel<TX, TY, NE>), dim3((unsigned)blocks), dim3(256), 0, a.stream,
                     static_cast<const TX*>(a.x), a.ldx ? a.ldx : a.d, a.branch, a.branch_f32, a.ldb ? a.ldb : a.d,
                     a.gamma, a.beta, a.resid_out, a.ldr ? a.ldr : a.d, static_cast<TY*>(a.y), a.ldy ? a.ldy : a.d,
                     a.rows, a.d, a.eps, a.row_mask, a.row_mask ? a.mask_resid : 0, a.row_mask ? a.mask_out : 0);
  return hipGetLastError();
}

template <typename TX, typename TY>
static hipError_t dispatch_ln_any(const LnArgs& a) {
  const int64_t ldy = a.ldy ? a.ldy : a.d;
  const int64_t w = ldy > a.d ? ldy : a.d;  // columns to write
  if (w <= 64) return launch_ln_any<TX, TY, 1>(a);
  if (w <= 128) return launch_ln_any<TX, TY, 2>(a);
  if (w <= 256) return launch_ln_any<TX, TY, 4>(a);
  if (w <= 512) return launch_ln_any<TX, TY, 8>(a);
  if (w <= 1024) return launch_ln_any<TX, TY, 16>(a);
  if (w <= 2048) return launch_ln_any<TX, TY, 32>(a);
  return launch_ln_any<TX, TY, 64>(a);
}

template <typename TX, typename TY, int NCH>
static hipError_t launch_ln_plain(const LnArgs& a) {
  const int64_t blocks = (a.rows + 3) / 4;
  const f16* br = static_cast<const f16*>(a.branch);
  auto kern = br ? ln_plain_kernel<TX, TY, NCH, true> : ln_plain_kernel<TX, TY, NCH, false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, a.stream, static_cast<const TX*>(a.x), br, a.gamma,
                     a.beta, static_cast<TY*>(a.y), a.rows, a.eps);
  return hipGetLastError();
}

template <typename TX, typename TY, int LPR, int NCH>
static hipError_t launch_ln(const LnArgs& a) {
  constexpr int RPB = 4 * (64 / LPR);  // rows per 256-thread block
  const int64_t blocks = (a.rows + RPB - 1) / RPB;
  hipLaunchKernelGGL((ln_rows_kernel<TX, TY, LPR, NCH>), dim3((unsigned)blocks), dim3(256), 0, a.stream,
                     static_cast<const TX*>(a.x), a.branch, a.branch_f32, a.gamma, a.beta, a.resid_out,
                     static_cast<TY*>(a.y), a.rows, a.d, a.eps, a.row_mask, a.row_mask ? a.mask_resid : 0,
                     a.row_mask ? a.mask_out : 0);
  return hipGetLastError();
}

template <typename TX, typename TY>
static hipError_t dispatch_ln_geometry(const LnArgs& a) {
  if ((!a.branch || !a.branch_f32) && !a.row_mask && !a.resid_out && a.rows <= (int64_t)4 * 0x7fffffff) {
    if (a.d == 512) return launch_ln_plain<TX, TY, 1>(a);
    if (a.d == 1024) return launch_ln_plain<TX, TY, 2>(a);
  }
  const int nch = a.d / 8;
  if (nch <= 4) return launch_ln<TX, TY, 4, 1>(a);
  if (nch <= 8) return launch_ln<TX, TY, 8, 1>(a);
  if (nch <= 16) return launch_ln<TX, TY, 16, 1>(a);
  if (nch <= 32) return launch_ln<TX, TY, 32, 1>(a);
  if (nch <= 64) return launch_ln<TX, TY, 64, 1>(a);
  if (nch <= 128) return launch_ln<TX, TY, 64, 2>(a);
  if (nch <= 256) return launch_ln<TX, TY, 64, 4>(a);
  return launch_ln<TX, TY, 64, 8>(a);
}

static bool vec_aligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Element types of x and y (fp16, fp32 or bf16 each); vec: the 16-byte-chunk kernels.
template <typename TX>
static hipError_t ln_by_y(const LnArgs& a, bool vec) {
  switch (a.y_dtype) {
    case kF16: return vec ? dispatch_ln_geometry<TX, f16>(a) : dispatch_ln_any<TX, f16>(a);
    case kF32: return vec ? dispatch_ln_geometry<TX, float>(a) : dispatch_ln_any<TX, float>(a);
    case kBF16: return vec ? dispatch_ln_geometry<TX, bf16>(a) : dispatch_ln_any<TX, bf16>(a);
    default: return hipErrorInvalidValue;
  }
}

hipError_t run_ln(const LnArgs& a) {
  if (a.rows < 0 || a.d <= 0 || a.d > kLnMaxD) return hipErrorInvalidValue;
  const int64_t d = a.d;
  if ((a.ldx && a.ldx < d) || (a.ldb && a.ldb < d) || (a.ldr && a.ldr < d) || (a.ldy && a.ldy < d))
    return hipErrorInvalidValue;
  if (a.rows == 0) return hipSuccess;
  // The vector kernels need whole 16-byte chunks: width a multiple of 8, dense rows,
  // 16-byte aligned buffers.
  const bool dense = (!a.ldx || a.ldx == d) && (!a.ldb || a.ldb == d) && (!a.ldr || a.ldr == d) && (!a.ldy || a.ldy == d);
  const bool vec = d % 8 == 0 && dense && vec_aligned(a.x) && vec_aligned(a.y) && (!a.branch || vec_aligned(a.branch)) &&
                   (!a.resid_out || vec_aligned(a.resid_out)) && (!a.gamma || vec_aligned(a.gamma)) &&
                   (!a.beta || vec_aligned(a.beta));
  switch (a.x_dtype) {
    case kF16: return ln_by_y<f16>(a, vec);
    case kF32: return ln_by_y<float>(a, vec);
    case kBF16: return ln_by_y<bf16>(a, vec);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace cobra
