// LayerNorm fused into the prologue of the projection that consumes it, for
// rows that fit one k-tile (d_model 64 or 128):
//
//   h = LayerNorm(x) * gamma + beta   (per row, fp32 statistics, biased variance)
//   c = h W^T + bias                  (fp16 operands, fp32 accumulate, fp16 out)
//
// The reference runs _add_ln_kernel and then the QKV GEMM (TTB:1216-1234), so
// h makes a round trip through HBM.  Here a workgroup normalises its 128 rows
// of x straight into the LDS tile the matrix cores read: h never exists in
// memory.  Row statistics use 8 or 16 lanes per row (DPP reductions); the
// normalised rows and the W tile sit row-major in LDS with 16-byte chunks
// XOR-swizzled by row, so every MFMA operand read is conflict-free.  The
// 128 x 128 fp16 result is staged back through the same LDS and written as
// whole 256-byte row segments (16 lanes per row), not as the 8-byte quads the
// accumulator layout would give.
#include "common.hpp"
#include "kernels.hpp"
#include "layer_common.hpp"
#include "lds_dma.hpp"

#include <type_traits>

namespace cobra {

namespace {

constexpr int kLgBM = 128, kLgBN = 128, kLgThreads = 256;

template <int D>
__device__ __forceinline__ int lg_swz(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);  // 16 / 8 chunks per row
}

// gamma / beta of 8 columns; null (LayerNorm without elementwise affine) reads
// as gamma 1, beta 0, which leaves the normalised value exact.
__device__ __forceinline__ void load_affine8(const float* gamma, const float* beta, int c0, float (&gv)[8],
                                             float (&bv)[8]) {
  if (gamma) {
    load8(gamma + c0, gv);
    load8(beta + c0, bv);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      gv[e] = 1.f;
      bv[e] = 0.f;
    }
  }
}

}  // namespace

template <int D, typename TX, typename TA>
__global__ __launch_bounds__(kLgThreads) void ln_gemm_kernel(const TX* __restrict__ x, const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, const TA* __restrict__ W,
                                                           const float* __restrict__ bias, TA* __restrict__ C,
                                                           int64_t M, int N, float eps) {
  using V8 = typename Op16<TA>::V8;
  using V4 = typename Op16<TA>::V4;
  static_assert(D == 64 || D == 128, "one k-tile per row");
  constexpr int ROWB = D * 2;               // bytes of one fp16 row
  constexpr int CPR = D / 8;                // 16-byte chunks per row (= lanes per row in the LN)
  constexpr int RPW = 64 / CPR;             // rows per wave per pass
  constexpr int PASSES = kLgBM / (4 * RPW);
  constexpr int WCH = kLgBN * CPR / kLgThreads;  // W chunks per thread
  constexpr int KS = D / 16;
  constexpr int OUTB = kLgBN * 2;           // bytes of one staged output row (128 fp16)
  constexpr int LDSB = (kLgBM + kLgBN) * ROWB > kLgBM * OUTB ? (kLgBM + kLgBN) * ROWB : kLgBM * OUTB;
  __shared__ __attribute__((aligned(16))) char smem[LDSB];
  char* const Hs = smem;
  char* const Ws = smem + kLgBM * ROWB;

  // Row blocks outermost, so the column tiles of a row block (which re-read the
  // same x rows) run next to each other on one XCD.
  const int nbn = (N + kLgBN - 1) / kLgBN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t m0 = (int64_t)(tile / nbn) * kLgBM;
  const int n0 = (tile % nbn) * kLgBN;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, g = lane >> 5;

  // ---- loads: the W tile (rows past N repeat row N-1; never stored) and x rows ------
  V8 wr[WCH];
#pragma unroll
  for (int i = 0; i < WCH; ++i) {
    const int c = tid + i * kLgThreads;
    const int r = c / CPR, ch = c % CPR;
    wr[i] = *reinterpret_cast<const V8*>(W + (int64_t)min(n0 + r, N - 1) * D + 8 * ch);
  }
  const int cl = lane % CPR;  // this lane's 8 columns: 8cl .. 8cl+7
  float xv[PASSES][8];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int r = (p * 4 + w) * RPW + lane / CPR;
    load8(x + min(m0 + r, M - 1) * D + 8 * cl, xv[p]);
  }
  float gv[8], bv[8];
  load_affine8(gamma, beta, 8 * cl, gv, bv);
#pragma unroll
  for (int i = 0; i < WCH; ++i) {
    const int c = tid + i * kLgThreads;
    const int r = c / CPR, ch = c % CPR;
    *reinterpret_cast<V8*>(Ws + r * ROWB + 16 * (ch ^ lg_swz<D>(r))) = wr[i];
  }
  // ---- LayerNorm of every row into the h tile ---------------------------------------
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const int r = (p * 4 + w) * RPW + lane / CPR;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += xv[p][e];
    const float mean = group_sum<CPR>(s) * (1.0f / D);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float t = xv[p][e] - mean;
      q += t * t;
    }
    const float rstd = rsqrtf(group_sum<CPR>(q) * (1.0f / D) + eps);
    V8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (TA)((xv[p][e] - mean) * rstd * gv[e] + bv[e]);
    *reinterpret_cast<V8*>(Hs + r * ROWB + 16 * (cl ^ lg_swz<D>(r))) = h;
  }
  __syncthreads();

  // ---- c^T tiles: wave (wm, wn) owns rows 64wm.., columns 64wn.. -------------------
  const int wm = w >> 1, wn = w & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 2; ++i) acc[j][i] = zero16();
  const int sw = lg_swz<D>(li);  // rows 32k + li share the swizzle of li
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int co = 16 * ((2 * kk + g) ^ sw);
    V8 af[2], wf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const V8*>(Hs + (64 * wm + 32 * i + li) * ROWB + co);
#pragma unroll
    for (int j = 0; j < 2; ++j) wf[j] = *reinterpret_cast<const V8*>(Ws + (64 * wn + 32 * j + li) * ROWB + co);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 2; ++i) acc[j][i] = mfma32x32x16(wf[j], af[i], acc[j][i]);
  }
  __syncthreads();  // every operand read is done: the LDS becomes the output staging tile

  // ---- + bias into a [128][128] fp16 staging tile (16-byte chunk c of row r at
  // c ^ (r & 15)), then whole row segments to C --------------------------------------------
  // lane li of (i, j) holds row 64wm + 32i + li, columns 64wn + 32j + 8q + 4g + {0..3}
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = 64 * wn + 32 * j + 8 * q + 4 * g;
      const int n = n0 + col;
      const f32x4 bq = (bias && n < N) ? *reinterpret_cast<const f32x4*>(bias + n) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = 64 * wm + 32 * i + li;
        V4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (TA)(acc[j][i][4 * q + e] + bq[e]);
        *reinterpret_cast<V4*>(smem + row * OUTB + 16 * ((col >> 3) ^ (row & 15)) + 8 * g) = o;
      }
    }
  __syncthreads();
  constexpr int CH = OUTB / 16;  // 16 chunks per staged row
#pragma unroll
  for (int it = 0; it < kLgBM * CH / kLgThreads; ++it) {
    const int idx = tid + it * kLgThreads;
    const int row = idx / CH, c = idx % CH;
    const int64_t m = m0 + row;
    const int n = n0 + 8 * c;
    if (m < M && n < N)  // N % 8 == 0: a chunk is all in or all out
      *reinterpret_cast<V8*>(C + m * N + n) = *reinterpret_cast<const V8*>(smem + row * OUTB + 16 * (c ^ (row & 15)));
  }
}

// ---------------------------------------------------------------------------------------
// The epilogue-side counterpart for short K (out-projection at d_model 64 / 128):
//   r = a W^T + bias (kEpiMaskBranch) + resid (kEpiMaskResid);  resid_out = r;
//   y = LayerNorm(r) * gamma + beta (kEpiMaskOut)
// with N = 64 or 128 columns (whole rows per workgroup) and K = 64 or 128 (one
// k-tile): the a and W tiles are loaded once, the fp32 product (+ bias) is staged
// in LDS, and a row pass of 16 lanes per row adds the residual, normalises and
// writes r and y as whole row segments.  Replaces _gemm_ln_kernel / _tl_linear_ln
// (TTB:394-488) for these shapes; its k loop and per-element residual loads are
// what the register-staged GEMM's LayerNorm epilogue spends its time on.
template <int K, int N, int BM, typename TR, typename TY, typename TA>
__global__ __launch_bounds__(kLgThreads) void gemm_ln_rows_kernel(
    const TA* __restrict__ A, const TA* __restrict__ W, const float* __restrict__ bias, const TR* __restrict__ resid,
    float* __restrict__ resid_out, const float* __restrict__ gamma, const float* __restrict__ beta, TY* __restrict__ Y,
    int64_t M, float eps, const uint8_t* __restrict__ row_mask, int epi) {
  using V8 = typename Op16<TA>::V8;
  static_assert((K == 64 || K == 128) && (N == 64 || N == 128), "one k-tile, whole rows");
  constexpr int ROWB = K * 2;
  constexpr int CPR = K / 8;
  constexpr int WM = BM >= 64 ? 2 : 1, WN = 4 / WM;  // waves over rows x columns
  constexpr int WTM = BM / WM, WTN = N / WN;         // wave tile
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  constexpr int ACH = BM * CPR / kLgThreads, WCH = N * CPR / kLgThreads;
  static_assert(ACH >= 1 && WCH >= 1 && ACH * kLgThreads == BM * CPR && WCH * kLgThreads == N * CPR, "loads");
  constexpr int LDC = N + 4;  // fp32 staging row stride
  constexpr int OPB = (BM + N) * ROWB, EPB = BM * LDC * 4;
  __shared__ __attribute__((aligned(16))) char smem[OPB > EPB ? OPB : EPB];
  char* const As = smem;
  char* const Ws = smem + BM * ROWB;
  float* const Cs = reinterpret_cast<float*>(smem);

  const int64_t m0 = (int64_t)xcd_remap(blockIdx.x, gridDim.x) * BM;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int li = lane & 31, g = lane >> 5;

  V8 ar[ACH], wr[WCH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = tid + i * kLgThreads;
    ar[i] = *reinterpret_cast<const V8*>(A + min(m0 + c / CPR, M - 1) * K + 8 * (c % CPR));
  }
#pragma unroll
  for (int i = 0; i < WCH; ++i) {
    const int c = tid + i * kLgThreads;
    wr[i] = *reinterpret_cast<const V8*>(W + (int64_t)(c / CPR) * K + 8 * (c % CPR));
  }
  // The residual chunks of the row pass below, requested now so that they arrive
  // under the products instead of after them.
  constexpr int LPR = N / 8, RPP = kLgThreads / LPR;
  static_assert(BM % RPP == 0, "row pass covers the block");
  const int cl = tid % LPR;
  RowChunk<TR> rr[BM / RPP];
  if (resid) {
#pragma unroll
    for (int it = 0; it < BM / RPP; ++it) {
      const int64_t m = m0 + it * RPP + tid / LPR;
      rr[it] = load_chunk(resid + (m < M ? m : M - 1) * N + 8 * cl);
    }
  }
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = tid + i * kLgThreads, r = c / CPR;
    *reinterpret_cast<V8*>(As + r * ROWB + 16 * ((c % CPR) ^ lg_swz<K>(r))) = ar[i];
  }
#pragma unroll
  for (int i = 0; i < WCH; ++i) {
    const int c = tid + i * kLgThreads, r = c / CPR;
    *reinterpret_cast<V8*>(Ws + r * ROWB + 16 * ((c % CPR) ^ lg_swz<K>(r))) = wr[i];
  }
  __syncthreads();

  const int wm = w / WN, wn = w % WN;
  f32x16 acc[TN][TM];
#pragma unroll
  for (int j = 0; j < TN; ++j)
#pragma unroll
    for (int i = 0; i < TM; ++i) acc[j][i] = zero16();
  const int sw = lg_swz<K>(li);
#pragma unroll
  for (int kk = 0; kk < K / 16; ++kk) {
    const int co = 16 * ((2 * kk + g) ^ sw);
    V8 af[TM], wf[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const V8*>(As + (wm * WTM + 32 * i + li) * ROWB + co);
#pragma unroll
    for (int j = 0; j < TN; ++j) wf[j] = *reinterpret_cast<const V8*>(Ws + (wn * WTN + 32 * j + li) * ROWB + co);
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[j][i] = mfma32x32x16(wf[j], af[i], acc[j][i]);
  }
  __syncthreads();  // operands are dead: the LDS becomes the fp32 staging tile

  // product + bias (padded rows' branch zeroed) into Cs[row][col]; lane li of (i, j) holds
  // row wm*WTM + 32i + li, columns wn*WTN + 32j + 8q + 4g + {0..3}
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = wm * WTM + 32 * i + li;
    const int64_t m = m0 + row;
    const bool zero = (epi & kEpiMaskBranch) && m < M && row_mask[m] == 0;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = wn * WTN + 32 * j + 8 * q + 4 * g;
        const f32x4 bq = bias ? *reinterpret_cast<const f32x4*>(bias + col) : f32x4{0.f, 0.f, 0.f, 0.f};
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = zero ? 0.f : acc[j][i][4 * q + e] + bq[e];
        *reinterpret_cast<f32x4*>(Cs + row * LDC + col) = v;
      }
  }
  __syncthreads();

  // row pass: LPR lanes per row, 8 consecutive columns per lane
  float gv[8], bv[8];
  load_affine8(gamma, beta, 8 * cl, gv, bv);
#pragma unroll
  for (int it = 0; it < BM / RPP; ++it) {
    const int row = it * RPP + tid / LPR;
    const int64_t m = m0 + row;
    const bool ok = m < M;
    float v[8], rv[8];
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(Cs + row * LDC + 8 * cl);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(Cs + row * LDC + 8 * cl + 4);
    if (resid) {
      to_float8(rr[it], rv);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) rv[e] = 0.f;
    }
    const float keep = (row_mask && ok && row_mask[m] == 0) ? 0.f : 1.f;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = (e < 4 ? c0[e] : c1[e - 4]) + rv[e];
      if (epi & kEpiMaskResid) v[e] *= keep;
      s += v[e];
    }
    const float mean = group_sum<LPR>(s) * (1.0f / N);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float t = v[e] - mean;
      q += t * t;
    }
    const float rstd = rsqrtf(group_sum<LPR>(q) * (1.0f / N) + eps);
    if (!ok) continue;
    if (resid_out) store8(resid_out + m * N + 8 * cl, v);
    const float ok_out = (epi & kEpiMaskOut) ? keep : 1.f;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = ((v[e] - mean) * rstd * gv[e] + bv[e]) * ok_out;
    store8(Y + m * N + 8 * cl, o);
  }
}

template <int K, int N, typename TR, typename TY, typename TA>
static hipError_t launch_gemm_ln_rows(const GemmArgs& a) {
  // The smallest block whose wave tiles are still 32 columns wide (32 rows at N = 128,
  // 64 at 64): several workgroups per CU in different phases, so that one's loads
  // overlap another's products.  (128-row blocks -- at B64 S1024 one round of 512
  // workgroups, all loading, then all computing -- measured 1.6 us slower there.)
  constexpr int SBM = N == 128 ? 32 : 64;
  const int64_t blocks = (a.M + SBM - 1) / SBM;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_ln_rows_kernel<K, N, SBM, TR, TY, TA>), dim3((unsigned)blocks), dim3(kLgThreads), 0,
                     a.stream, static_cast<const TA*>(a.a), static_cast<const TA*>(a.w), a.bias,
                     static_cast<const TR*>(a.resid), static_cast<float*>(a.c), a.ln_gamma, a.ln_beta,
                     static_cast<TY*>(a.ln_y), a.M, a.eps, a.row_mask, a.epi);
  return hipGetLastError();
}

template <typename TR, typename TY, typename TA>
static hipError_t gemm_ln_rows_shape(const GemmArgs& a) {
  if (a.K == 128)
    return a.N == 128 ? launch_gemm_ln_rows<128, 128, TR, TY, TA>(a) : launch_gemm_ln_rows<128, 64, TR, TY, TA>(a);
  return a.N == 128 ? launch_gemm_ln_rows<64, 128, TR, TY, TA>(a) : launch_gemm_ln_rows<64, 64, TR, TY, TA>(a);
}

// Operands fp16 or bf16; y and the residual in the operand type or fp32.
bool gemm_ln_rows_ok(const GemmArgs& a) {
  const int op = a.ab_dtype;
  return a.ln_gamma && a.ln_beta && a.ln_y && (a.K == 64 || a.K == 128) && (a.N == 64 || a.N == 128) &&
         !(a.epi & kEpiGelu) && (!a.c || a.c_dtype == kF32) && (op == kF16 || op == kBF16) &&
         (a.ln_y_dtype == op || a.ln_y_dtype == kF32) && (!a.resid || a.resid_dtype == op || a.resid_dtype == kF32);
}

template <typename TA>
static hipError_t gemm_ln_rows_typed(const GemmArgs& a) {
  const bool y16 = a.ln_y_dtype != kF32;
  if (!a.resid || a.resid_dtype == kF32)
    return y16 ? gemm_ln_rows_shape<float, TA, TA>(a) : gemm_ln_rows_shape<float, float, TA>(a);
  return y16 ? gemm_ln_rows_shape<TA, TA, TA>(a) : gemm_ln_rows_shape<TA, float, TA>(a);
}

hipError_t run_gemm_ln_rows(const GemmArgs& a) {
  if (!gemm_ln_rows_ok(a)) return hipErrorInvalidValue;
  if (a.M == 0) return hipSuccess;
  return a.ab_dtype == kBF16 ? gemm_ln_rows_typed<bf16>(a) : gemm_ln_rows_typed<f16>(a);
}

// ---------------------------------------------------------------------------------------
// Persistent form for d_model 128 and N = 128 NT columns (the QKV projection: N = 384):
// a workgroup per CU keeps all of W in LDS and walks blocks of BM rows, so W is read
// once per CU rather than once per tile, and the rows two blocks ahead are loaded into
// registers while the current block's products and stores run.  Wave w owns output columns
// 128 t + 32 w .. + 31 (t < NT) of every block (NT x BM/32 accumulators, started from the
// bias); the results leave through LDS as whole row segments.  The tile-per-workgroup
// kernel above serialises load, LayerNorm, products and stores inside each workgroup,
// two per CU.  Operands (normalised rows, W, output) fp16 or bf16 (TA).
//
// NWV waves: with 8, waves w and w + 4 own the same columns and split the block's
// row tiles, so twice the loads and stores are in flight per CU (all of W in LDS
// leaves room for one workgroup per CU, and the kernel is bound by how many
// memory operations that workgroup keeps outstanding).
template <int NT, int BM, int NWV, typename TX, typename TA>
__global__ __launch_bounds__(64 * NWV) void ln_gemm_p_kernel(const TX* __restrict__ x, const float* __restrict__ gamma,
                                                           const float* __restrict__ beta, const TA* __restrict__ W,
                                                           const float* __restrict__ bias, TA* __restrict__ C,
                                                           int64_t M, float eps) {
  using V8 = typename Op16<TA>::V8;
  using V4 = typename Op16<TA>::V4;
  constexpr int D = 128, ROWB = 2 * D, CPR = D / 8;  // 16 chunks of 16 bytes per row
  constexpr int N = 128 * NT;
  constexpr int THREADS = 64 * NWV;
  constexpr int CG = NWV / 4;                         // wave groups splitting the row tiles
  constexpr int RT = BM / 32 / CG;                    // 32-row tiles per wave
  constexpr int PASSES = BM * CPR / THREADS;          // LayerNorm rows per thread
  constexpr int RPP = THREADS / CPR;                  // rows per LayerNorm pass
  constexpr int WCH = N * CPR / THREADS;              // W chunks per thread
  static_assert(NWV == 4 || NWV == 8 || NWV == 16, "four column groups of waves, one, two or four row groups");
  static_assert(BM % (32 * CG) == 0 && RT >= 1 && PASSES >= 1 && PASSES * THREADS == BM * CPR, "block rows");
  constexpr int SG = WCH % 4 == 0 ? 4 : 2;           // W chunks per staging group
  static_assert(WCH * THREADS == N * CPR && WCH % SG == 0, "W staging");
  __shared__ __attribute__((aligned(16))) char smem[N * ROWB + 2 * BM * ROWB];
  char* const Ws = smem;
  char* const Hs = smem + N * ROWB;  // two buffers of BM normalised rows

  const int tid = threadIdx.x;
  const int lane = tid & 63, w4 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int w = w4 % 4, rg = w4 / 4;         // column group, row group of this wave
  const int li = lane & 31, g = lane >> 5;
  const int rp = tid / CPR, cl = tid % CPR;  // LayerNorm: row rp of each RPP-row pass, chunk cl
  const int64_t nblk = (M + BM - 1) / BM;

  // W rows, swizzled: chunk c of row r at c ^ (r & 15).
#pragma unroll
  for (int b0 = 0; b0 < WCH; b0 += SG) {
    V8 v[SG];
#pragma unroll
    for (int i = 0; i < SG; ++i) {
      const int c = tid + THREADS * (b0 + i);
      v[i] = *reinterpret_cast<const V8*>(W + (int64_t)(c / CPR) * D + 8 * (c % CPR));
    }
#pragma unroll
    for (int i = 0; i < SG; ++i) {
      const int c = tid + THREADS * (b0 + i), r = c / CPR;
      *reinterpret_cast<V8*>(Ws + r * ROWB + 16 * ((c % CPR) ^ (r & 15))) = v[i];
    }
  }
  float gv[8], bv[8];
  load_affine8(gamma, beta, 8 * cl, gv, bv);
  // Bias of this wave's columns in the accumulator layout: tile t, register r ->
  // column 128 t + 32 w + 8 (r / 4) + 4 g + r % 4 (tile t of the four column waves
  // together covers the 128 columns 128 t .. 128 t + 127: q, k, v at N = 384).
  f32x16 bt[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = 128 * t + 32 * w + 8 * q + 4 * g;
      const f32x4 b4 = bias ? *reinterpret_cast<const f32x4*>(bias + n) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) bt[t][4 * q + e] = b4[e];
    }

  // Rows of block `blk` for this thread's LayerNorm slots, as loaded.  Two register
  // slots: the rows of block n + 2 are requested while block n's products and stores
  // run, so a block's loads have two blocks' time to land.  Rows past M (and blocks
  // past the last) load row M - 1, never stored: a load on every path, so that the
  // compiler's wait for a slot counts only the memory operations issued after it
  // (a zero fill on some paths made it wait for every store at the loop head).
  RowChunk<TX> xr[2][PASSES];
  auto load_rows = [&](RowChunk<TX>(&dst)[PASSES], int64_t blk) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int64_t row = blk * BM + RPP * p + rp;
      dst[p] = load_chunk(x + (row < M ? row : M - 1) * D + 8 * cl);
    }
  };
  const int64_t G = gridDim.x;
  load_rows(xr[0], blockIdx.x);
  asm volatile("" ::: "memory");
  load_rows(xr[1], blockIdx.x + G);
  // Slot 0 landed before the loop: the loop head's wait then only has to cover the
  // back edge, where slot 0's loads are followed by a whole block's stores and
  // slot 1's loads (otherwise the compiler's wait there, sized for this entry
  // path, drains most of the previous block's stores every second block).
  wait_vmcnt<PASSES * (int)(sizeof(RowChunk<TX>) / 16)>();

  // One block: LayerNorm of its rows (from slot S) into H buffer S, products, stores.
  auto block = [&](auto slot, int64_t blk) {
    constexpr int S = decltype(slot)::value;
    char* const H = Hs + S * BM * ROWB;
    // ---- LayerNorm of the block's rows into H ----------------------------------------
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      float xv[8];
      to_float8(xr[S][p], xv);
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s += xv[e];
      const float mean = group_sum<CPR>(s) * (1.0f / D);
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = xv[e] - mean;
        q += t * t;
      }
      const float rstd = rsqrtf(group_sum<CPR>(q) * (1.0f / D) + eps);
      V8 h;
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = (TA)((xv[e] - mean) * rstd * gv[e] + bv[e]);
      const int r = RPP * p + rp;
      *reinterpret_cast<V8*>(H + r * ROWB + 16 * (cl ^ (r & 15))) = h;
    }
    // One barrier per block: H of this block is complete, and (double buffering)
    // every wave finished the previous block's reads of the other buffer.
    __syncthreads();
    load_rows(xr[S], blk + 2 * G);

    // ---- products: NT column tiles x RT row tiles per wave ----------------------------
    f32x16 acc[NT][RT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < RT; ++i) acc[t][i] = bt[t];
    const int sw = li & 15;  // rows 32i + li and 128t + 32w + li share this swizzle
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      const int co = 16 * ((2 * kk + g) ^ sw);
      V8 hf[RT], wf[NT];
#pragma unroll
      for (int i = 0; i < RT; ++i) hf[i] = *reinterpret_cast<const V8*>(H + (32 * (RT * rg + i) + li) * ROWB + co);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wf[t] = *reinterpret_cast<const V8*>(Ws + (128 * t + 32 * w + li) * ROWB + co);
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < RT; ++i) acc[t][i] = mfma32x32x16(wf[t], hf[i], acc[t][i]);
    }

    // ---- fp16 out through LDS, one 128-column slab (tile t of every wave) at a time:
    // the slab's BM rows x 256 bytes go to an H buffer (chunk c of row r at c ^ (r & 15)),
    // then leave as whole 256-byte row segments, 16 lanes per row.  Written straight
    // from the accumulator layout, every store instruction would touch 32 rows with
    // 32 bytes each, which ran the projection at ~1/3 of the copy rate.  Slabs 0 and 2
    // use this block's H buffer, slab 1 the other one (free: the previous block is
    // done with it, and the next block's LayerNorm into it comes after slab 2's barrier).
    __syncthreads();  // every wave is done reading H for the products
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      char* const O = Hs + ((S + t) & 1) * BM * ROWB;
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        const int r = 32 * (RT * rg + i) + li;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          V4 h;
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = (TA)acc[t][i][4 * q + e];
          *reinterpret_cast<V4*>(O + r * ROWB + 16 * ((4 * w + q) ^ (r & 15)) + 8 * g) = h;
        }
      }
      __syncthreads();
      // Rows past M hold row M - 1's x, hence row M - 1's output: they store it there
      // again (unconditional stores keep the compiler's memory waits exact).
#pragma unroll
      for (int k = 0; k < BM * CPR / THREADS; ++k) {
        const int idx = tid + THREADS * k, r = idx / CPR, c = idx % CPR;
        const int64_t m = blk * BM + r;
        *reinterpret_cast<V8*>(C + (m < M ? m : M - 1) * N + 128 * t + 8 * c) =
            *reinterpret_cast<const V8*>(O + r * ROWB + 16 * (c ^ (r & 15)));
      }
      // No barrier here: slab t + 1 goes to the other buffer, and slab t + 2, which
      // reuses this one, is written after the barrier that follows slab t + 1's
      // writes, which every wave reaches only after its reads of slab t.
    }
  };
  for (int64_t blk = blockIdx.x; blk < nblk; blk += 2 * G) {
    block(std::integral_constant<int, 0>{}, blk);
    if (blk + G >= nblk) break;
    block(std::integral_constant<int, 1>{}, blk + G);
  }
}

template <int NT, typename TX, typename TA>
static hipError_t launch_ln_gemm_p(const LnGemmArgs& a) {
  const int64_t cus = compute_units();
  if (a.M >= (int64_t)64 * 2 * cus) {
    const int64_t nblk = (a.M + 63) / 64;
    hipLaunchKernelGGL((ln_gemm_p_kernel<NT, 64, 8, TX, TA>), dim3((unsigned)(nblk < cus ? nblk : cus)), dim3(512), 0,
                       a.stream, static_cast<const TX*>(a.x), a.gamma, a.beta, static_cast<const TA*>(a.w), a.bias,
                       static_cast<TA*>(a.c), a.M, a.eps);
  } else {
    const int64_t nblk = (a.M + 31) / 32;
    hipLaunchKernelGGL((ln_gemm_p_kernel<NT, 32, 4, TX, TA>), dim3((unsigned)(nblk < cus ? nblk : cus)),
                       dim3(kLgThreads), 0, a.stream, static_cast<const TX*>(a.x), a.gamma, a.beta,
                       static_cast<const TA*>(a.w), a.bias, static_cast<TA*>(a.c), a.M, a.eps);
  }
  return hipGetLastError();
}

template <int D, typename TX, typename TA>
static hipError_t launch_ln_gemm(const LnGemmArgs& a) {
  const int64_t tiles = ((a.M + kLgBM - 1) / kLgBM) * (int64_t)((a.N + kLgBN - 1) / kLgBN);
  if (tiles > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((ln_gemm_kernel<D, TX, TA>), dim3((unsigned)tiles), dim3(kLgThreads), 0, a.stream,
                     static_cast<const TX*>(a.x), a.gamma, a.beta, static_cast<const TA*>(a.w), a.bias,
                     static_cast<TA*>(a.c), a.M, a.N, a.eps);
  return hipGetLastError();
}

template <typename TX, typename TA>
static hipError_t ln_gemm_typed(const LnGemmArgs& a) {
  if (a.d == 128 && a.N == 384) return launch_ln_gemm_p<3, TX, TA>(a);
  return a.d == 128 ? launch_ln_gemm<128, TX, TA>(a) : launch_ln_gemm<64, TX, TA>(a);
}

// fp16 operands with fp16 or fp32 x; bf16 operands with bf16 or fp32 x.
bool ln_gemm_ok(int64_t d, int x_dtype, int ab_dtype) {
  if (d != 64 && d != 128) return false;
  if (ab_dtype == kBF16) return x_dtype == kBF16 || x_dtype == kF32;
  return ab_dtype == kF16 && (x_dtype == kF16 || x_dtype == kF32);
}

hipError_t run_ln_gemm(const LnGemmArgs& a) {
  if (!ln_gemm_ok(a.d, a.x_dtype, a.ab_dtype) || a.M < 0 || a.N <= 0 || a.N % 8 != 0 || a.N > 3 * a.d)
    return hipErrorInvalidValue;
  if (!a.x || !a.w || !a.c || (a.gamma == nullptr) != (a.beta == nullptr)) return hipErrorInvalidValue;
  if (a.M == 0) return hipSuccess;
  if (a.ab_dtype == kBF16) return a.x_dtype == kBF16 ? ln_gemm_typed<bf16, bf16>(a) : ln_gemm_typed<float, bf16>(a);
  return a.x_dtype == kF16 ? ln_gemm_typed<f16, f16>(a) : ln_gemm_typed<float, f16>(a);
}

}  // namespace cobra
