// C[M,N] = A[M,K] . W[N,K]^T (+ bias[N]) (+ resid[M,N]), fp16 or bf16 operands, fp32
// accumulate, with an optional LayerNorm epilogue over whole rows (fp16 operands).
//
// Replaces the reference's _gemm_kernel/_tl_linear (torch_transformer_benchmark.py:283-381)
// for the projections and _gemm_ln_kernel/_tl_linear_ln (TTB:394-488) for
// out_proj + bias + residual -> fp32 residual -> LayerNorm.  Epilogue options
// (kEpi* flags, in this order): exact GELU, padded rows' branch set to 0
// (masked_fill before the residual add), residual add, padded rows' sum
// multiplied by 0 (the reference's MASK_RESID), and in the LayerNorm epilogue
// the padded rows' output multiplied by 0 (MASK_OUT).  Same ownership
// invariant as the reference: every output element belongs to exactly one
// workgroup, there is no split-K and no atomics, so results are bit-repeatable.
//
// W stays in nn.Linear's [N, K] layout: both operands are k-contiguous, which
// is exactly what a 32x32x16 MFMA operand wants (8 consecutive k per lane, one
// 16-byte LDS read), so no transposed weight copy is ever made.
//
// Pipeline: BM x BN x 64 tiles in LDS (rows padded by 16 B, conflict-free for
// ds_read_b128), the next k-tile prefetched into registers while the current
// one feeds the matrix cores.
#include "common.hpp"
#include "kernels.hpp"

namespace cobra {

template <int BM, int BN, int WM, int WN>
struct GemmTile {
  static constexpr int BK = 64;
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM;  // wave tile rows
  static constexpr int WTN = BN / WN;  // wave tile cols
  static constexpr int TM = WTM / 32;  // MFMA tiles per wave (rows)
  static constexpr int TN = WTN / 32;
  static constexpr int LDK = BK + 8;   // halves per LDS row
  static constexpr int A_IT = BM * (BK / 8) / NT;
  static constexpr int W_IT = BN * (BK / 8) / NT;
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32x32 MFMA tile");
  static_assert(A_IT * NT == BM * (BK / 8) && W_IT * NT == BN * (BK / 8), "tile loads must divide evenly");
};

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return (float)v;
}

// 1 for a valid row, 0 for a padded one.
__device__ __forceinline__ float row_valid(const uint8_t* __restrict__ mask, int64_t m) {
  return mask[m] != 0 ? 1.f : 0.f;
}

// The epilogue steps between the bias and the residual add.
__device__ __forceinline__ float epi_pre_resid(float v, int epi, const uint8_t* __restrict__ mask, int64_t m) {
  if (epi & kEpiGelu) v = gelu_erf(v);
  if ((epi & kEpiMaskBranch) && mask[m] == 0) v = 0.f;
  return v;
}

template <int BM, int BN, int WM, int WN, typename TR, typename TC, bool LN_EPI, typename TY, typename TA>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(const TA* __restrict__ A, const TA* __restrict__ W,
                                                          const float* __restrict__ bias, const TR* __restrict__ resid,
                                                          TC* __restrict__ C, int64_t M, int N, int K,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, TY* __restrict__ Y,
                                                          float eps, const uint8_t* __restrict__ row_mask, int epi) {
  using T = GemmTile<BM, BN, WM, WN>;
  constexpr int BK = T::BK, LDK = T::LDK, NT = T::NT;
  constexpr int GEMM_LDS = (BM + BN) * LDK * 2;
  constexpr int LDC = BN + 4;  // fp32 staging row stride for the LN epilogue
  constexpr int EPI_LDS = LN_EPI ? BM * LDC * 4 : 0;
  constexpr int LDS_BYTES = GEMM_LDS > EPI_LDS ? GEMM_LDS : EPI_LDS;
  __shared__ __attribute__((aligned(16))) char smem[LDS_BYTES];
  using V8 = typename Op16<TA>::V8;
  TA* As = reinterpret_cast<TA*>(smem);
  TA* Ws = As + BM * LDK;

  const int nbn = (N + BN - 1) / BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t m0 = (int64_t)(tile / nbn) * BM;
  const int n0 = (tile % nbn) * BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, g = lane >> 5;

  V8 ra[T::A_IT], rw[T::W_IT];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < T::A_IT; ++i) {
      const int c = tid + i * NT;
      const int64_t m = m0 + c / (BK / 8);
      const int k = k0 + (c % (BK / 8)) * 8;
      ra[i] = (m < M && k < K) ? *reinterpret_cast<const V8*>(A + m * K + k) : zero8_of<TA>();
    }
#pragma unroll
    for (int i = 0; i < T::W_IT; ++i) {
      const int c = tid + i * NT;
      const int n = n0 + c / (BK / 8);
      const int k = k0 + (c % (BK / 8)) * 8;
      rw[i] = (n < N && k < K) ? *reinterpret_cast<const V8*>(W + (int64_t)n * K + k) : zero8_of<TA>();
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < T::A_IT; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<V8*>(As + (c / (BK / 8)) * LDK + (c % (BK / 8)) * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < T::W_IT; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<V8*>(Ws + (c / (BK / 8)) * LDK + (c % (BK / 8)) * 8) = rw[i];
    }
  };

  f32x16 acc[T::TM][T::TN];
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) acc[i][j] = zero16();

  const int KT = (K + BK - 1) / BK;
  gload(0);
  sstore();
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const bool more = kt + 1 < KT;
    if (more) gload((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      V8 af[T::TM], bf[T::TN];
#pragma unroll
      for (int i = 0; i < T::TM; ++i)
        af[i] = *reinterpret_cast<const V8*>(As + (wm * T::WTM + i * 32 + li) * LDK + kk * 16 + g * 8);
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
        bf[j] = *reinterpret_cast<const V8*>(Ws + (wn * T::WTN + j * 32 + li) * LDK + kk * 16 + g * 8);
#pragma unroll
      for (int i = 0; i < T::TM; ++i)
#pragma unroll
        for (int j = 0; j < T::TN; ++j) acc[i][j] = mfma32x32x16(af[i], bf[j], acc[i][j]);
    }
    __syncthreads();
    if (more) {
      sstore();
      __syncthreads();
    }
  }

  if constexpr (!LN_EPI) {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) {
        const int n = n0 + wn * T::WTN + j * 32 + li;
        const float bn = (bias && n < N) ? bias[n] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = m0 + wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (m < M && n < N) {
            float v = acc[i][j][r] + bn;
            if (epi) v = epi_pre_resid(v, epi, row_mask, m);
            if (resid) v += to_f32(resid[m * N + n]);
            if (epi & kEpiMaskResid) v *= row_valid(row_mask, m);
            C[m * N + n] = (TC)v;
          }
        }
      }
  } else {
    // Stage the fp32 tile (+ bias + residual) in LDS, then normalise whole rows:
    // 16 lanes per row, 8-element chunks per lane.  The GEMM's LDS is free here
    // (the k-loop ended on a barrier).
    float* Cs = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) {
        const int col = wn * T::WTN + j * 32 + li;
        const float bn = (bias && col < N) ? bias[col] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          const int64_t m = m0 + row;
          float v = acc[i][j][r] + bn;
          if (m < M && col < N) {
            if (epi) v = epi_pre_resid(v, epi, row_mask, m);
            if (resid) v += to_f32(resid[m * N + col]);
            if (epi & kEpiMaskResid) v *= row_valid(row_mask, m);
          }
          Cs[row * LDC + col] = v;
        }
      }
    __syncthreads();

    constexpr int CPL = BN / 16 / 8;  // 8-element chunks per lane
    static_assert(CPL >= 1 && BM % (NT / 16) == 0, "LN epilogue geometry");
    const int nch = N >> 3;
    for (int rr = tid / 16; rr < BM; rr += NT / 16) {
      const int64_t m = m0 + rr;
      float v[CPL][8];
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = (tid % 16) + c * 16;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[c][e] = ch < nch ? Cs[rr * LDC + ch * 8 + e] : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[c][e];
      }
      const float mean = group_sum<16>(s) / (float)N;
      float q = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c)
        if ((tid % 16) + c * 16 < nch)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float t = v[c][e] - mean;
            q += t * t;
          }
      const float rstd = rsqrtf(group_sum<16>(q) / (float)N + eps);
      if (m < M) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int ch = (tid % 16) + c * 16;
          if (ch >= nch) continue;
          if (C) store8(reinterpret_cast<float*>(C) + m * N + ch * 8, v[c]);
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (v[c][e] - mean) * rstd * gamma[ch * 8 + e] + beta[ch * 8 + e];
          if (epi & kEpiMaskOut) {
            const float mv = row_valid(row_mask, m);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] *= mv;
          }
          store8(Y + m * N + ch * 8, o);
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, typename TR, typename TC, bool LN_EPI, typename TY, typename TA = f16>
static hipError_t launch_gemm(const GemmArgs& a) {
  const int64_t tiles = ((a.M + BM - 1) / BM) * (int64_t)((a.N + BN - 1) / BN);
  if (tiles > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, TR, TC, LN_EPI, TY, TA>), dim3((unsigned)tiles), dim3(WM * WN * 64),
                     0, a.stream, static_cast<const TA*>(a.a), static_cast<const TA*>(a.w), a.bias,
                     static_cast<const TR*>(a.resid), static_cast<TC*>(a.c), a.M, a.N, a.K, a.ln_gamma, a.ln_beta,
                     static_cast<TY*>(a.ln_y), a.eps, a.row_mask, a.epi);
  return hipGetLastError();
}

// Plain epilogue: pick the row tile so that the grid still covers the chip.
template <typename TR, typename TC, typename TA = f16>
static hipError_t dispatch_plain(const GemmArgs& a) {
  const int64_t big = ((a.M + 127) / 128) * (int64_t)((a.N + 127) / 128);
  if (big >= 512) return launch_gemm<128, 128, 2, 2, TR, TC, false, f16, TA>(a);
  return launch_gemm<64, 128, 2, 2, TR, TC, false, f16, TA>(a);
}

// bf16 operands: plain epilogue, residual bf16 or fp32, output bf16 or fp32.
static hipError_t run_gemm_bf16(const GemmArgs& a) {
  if (a.ln_gamma) return gemm_ln_rows_ok(a) ? run_gemm_ln_rows(a) : hipErrorInvalidValue;  // K, N in {64, 128}
  if (!a.c) return hipErrorInvalidValue;
  const bool rb = !a.resid || a.resid_dtype == kBF16;
  if (!rb && a.resid_dtype != kF32) return hipErrorInvalidValue;
  if (a.c_dtype != kBF16 && a.c_dtype != kF32) return hipErrorInvalidValue;
  if (gemm_dma_ok(a)) return run_gemm_dma(a);
  if (a.c_dtype == kBF16) return rb ? dispatch_plain<bf16, bf16, bf16>(a) : dispatch_plain<float, bf16, bf16>(a);
  return rb ? dispatch_plain<bf16, float, bf16>(a) : dispatch_plain<float, float, bf16>(a);
}

template <typename TR, typename TY>
static hipError_t dispatch_ln(const GemmArgs& a) {
  // One column block owns the whole row; 32-row tiles keep >= 256 workgroups
  // down to M = 8192.
  if (a.M >= 64 * 512) return launch_gemm<64, 128, 2, 2, TR, float, true, TY>(a);
  return launch_gemm<32, 128, 1, 4, TR, float, true, TY>(a);
}

hipError_t run_gemm(const GemmArgs& a) {
  if (a.M < 0 || a.N <= 0 || a.K <= 0 || a.K % 8 != 0) return hipErrorInvalidValue;
  if (!a.a || !a.w) return hipErrorInvalidValue;
  if ((a.epi & ~(kEpiGelu | kEpiMaskBranch | kEpiMaskResid | kEpiMaskOut)) != 0) return hipErrorInvalidValue;
  if ((a.epi & (kEpiMaskBranch | kEpiMaskResid | kEpiMaskOut)) && !a.row_mask) return hipErrorInvalidValue;
  if ((a.epi & kEpiMaskOut) && !a.ln_gamma) return hipErrorInvalidValue;
  if (a.M == 0) return hipSuccess;
  if (a.ab_dtype == kBF16) return run_gemm_bf16(a);
  if (a.ab_dtype != kF16) return hipErrorInvalidValue;
  const bool has_resid = a.resid != nullptr;
  if (has_resid && a.resid_dtype != kF16 && a.resid_dtype != kF32) return hipErrorInvalidValue;
  if (a.ln_gamma && gemm_ln_rows_ok(a)) return run_gemm_ln_rows(a);
  if (a.ln_gamma) {
    if (!a.ln_beta || !a.ln_y || a.N > 128 || a.N % 8 != 0) return hipErrorInvalidValue;
    if (a.c && a.c_dtype != kF32) return hipErrorInvalidValue;
    const bool y16 = a.ln_y_dtype == kF16;
    if (!y16 && a.ln_y_dtype != kF32) return hipErrorInvalidValue;
    if (!has_resid || a.resid_dtype == kF32)
      return y16 ? dispatch_ln<float, f16>(a) : dispatch_ln<float, float>(a);
    return y16 ? dispatch_ln<f16, f16>(a) : dispatch_ln<f16, float>(a);
  }
  if (!a.c) return hipErrorInvalidValue;
  const bool c16 = a.c_dtype == kF16;
  if (!c16 && a.c_dtype != kF32) return hipErrorInvalidValue;
  if (gemm_dma_ok(a)) return run_gemm_dma(a);
  if (!has_resid || a.resid_dtype == kF16) return c16 ? dispatch_plain<f16, f16>(a) : dispatch_plain<f16, float>(a);
  return c16 ? dispatch_plain<float, f16>(a) : dispatch_plain<float, float>(a);
}

}  // namespace cobra
