// C[M,N] = A[M,K] . W[N,K]^T (+ bias[N]) (+ resid[M,N]) for the large
// projections: fp16 or bf16 operands, fp32 accumulate, C in the operand type or fp32.
//
// Same contract as the register-staged GEMM (replaces the reference's
// _gemm_kernel / _tl_linear, torch_transformer_benchmark.py:283-381): each
// output element is owned by exactly one workgroup, no split-K, no atomics.
//
// gfx950 mapping:
//   * operand tiles move HBM/L2 -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging, no ds_write): one wave instruction fills one contiguous 1 KB
//     band = 8 rows of a 64-wide k-tile.  The LDS tile is XOR-swizzled in
//     16-byte chunks (chunk c of row r at c ^ ((r >> 1) & 7)); since the DMA
//     destination of a lane is fixed (band base + 16 * lane), each lane instead
//     fetches the global chunk that belongs in its slot;
//   * ST stages of LDS, one barrier per k-tile: a wave waits for its own DMA
//     of tile kt (vmcnt), the barrier makes every wave's DMA visible and
//     retires the stage computed in the previous step, which then receives
//     tile kt + ST - 1;
//   * v_mfma_f32_32x32x16_f16 (_bf16) with the weight tile as the A operand, so the
//     accumulator holds C^T: each lane owns one output row and 4 consecutive
//     columns per register quad;
//   * epilogue through LDS: the fp32 tile (+ bias) is staged, then written in
//     whole-row, 16-byte-per-lane passes with the kEpi* options (GELU, row
//     masks) and the residual applied on the way.
#include "common.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace cobra {

namespace {

template <int BM, int BN, int WM, int WN, int ST>
struct DmaTile {
  // (GM, the tile-order group height, is a kernel parameter of its own.)
  static constexpr int BK = 64;
  static constexpr int NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int ROWS = BM + BN;          // LDS rows per stage: A rows, then W rows
  static constexpr int STAGE = ROWS * BK;       // halves per stage
  static constexpr int BANDS = ROWS / 8;        // 1 KB bands per stage
  static constexpr int LPT = BANDS / NW;        // DMA instructions per thread per k-tile
  static constexpr int EPW = WN * 32;           // epilogue slice width: one 32-column block per wave column
  static constexpr int LDC = EPW + 4;           // fp32 epilogue row stride (floats)
  static constexpr int GEMM_LDS = ST * STAGE * 2;
  static constexpr int EPI_LDS = BM * LDC * 4;
  static constexpr int LDS = GEMM_LDS > EPI_LDS ? GEMM_LDS : EPI_LDS;
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  static_assert(BANDS % NW == 0, "every wave issues the same number of DMA bands");
  static_assert(BM % 16 == 0 && BN % 16 == 0, "swizzle period");
  static_assert(LDS <= 163840, "LDS budget");
};

__device__ __forceinline__ int chunk_swz(int row) { return (row >> 1) & 7; }

template <typename T>
__device__ __forceinline__ float to_float(T v) {
  return (float)v;
}

}  // namespace

// The k-loop of the LDS-DMA GEMMs: acc[j][i] += (W rows n0 + wn*WTN + 32j ..) x
// (A rows m0 + wm*WTM + 32i ..)^T over all of K.
template <int BM, int BN, int WM, int WN, int ST, typename TA>
__device__ __forceinline__ void dma_mainloop(const TA* __restrict__ A, const TA* __restrict__ W, int64_t M, int N,
                                             int K, int64_t m0, int n0, char* smem,
                                             f32x16 (&acc)[BN / WN / 32][BM / WM / 32]) {
  using T = DmaTile<BM, BN, WM, WN, ST>;
  constexpr int BK = T::BK, NW = T::NW, LPT = T::LPT;
  using V8 = typename Op16<TA>::V8;
  const TA* lds = reinterpret_cast<const TA*>(smem);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, g = lane >> 5;

  // DMA sources.  Band b = wave + i * NW covers stage rows 8b..8b+7; this lane
  // fills row 8b + lane/8, slot lane%8, i.e. logical chunk slot ^ swz(row).
  // Rows past M or N are clamped to the last valid row: their products land in
  // accumulator entries that are never stored.
  const TA* Ablk = A + m0 * K;
  const TA* Wblk = W + (int64_t)n0 * K;
  unsigned src_off[LPT];  // bytes from the block base (A rows) or W block base
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int row = 8 * (wave + i * NW) + (lane >> 3);
    const int chunk = (lane & 7) ^ chunk_swz(row);
    if (row < BM) {
      const int64_t m = min(m0 + row, M - 1) - m0;
      src_off[i] = (unsigned)((m * K + chunk * 8) * 2);
    } else {
      const int n = min(n0 + row - BM, N - 1) - n0;
      src_off[i] = (unsigned)(((int64_t)n * K + chunk * 8) * 2);
    }
  }
  auto issue = [&](int stage, int k0) {
    char* sbase = smem + stage * T::STAGE * 2;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int band = wave + i * NW;
      const char* src = (8 * band < BM ? reinterpret_cast<const char*>(Ablk) : reinterpret_cast<const char*>(Wblk)) +
                        (int64_t)k0 * 2 + src_off[i];
      dma16(src, sbase + band * 1024);
    }
  };

#pragma unroll
  for (int j = 0; j < T::TN; ++j)
#pragma unroll
    for (int i = 0; i < T::TM; ++i) acc[j][i] = zero16();

  // Operand rows of this lane: A rows wm*WTM + i*32 + li, W rows BM + wn*WTN + j*32 + li;
  // all share swz = (li >> 1) & 7 (tile offsets are multiples of 16).
  const int sw = chunk_swz(li);
  const int arow = (wm * T::WTM + li) * BK;
  const int wrow = (BM + wn * T::WTN + li) * BK;

  const int KT = K / BK;
#pragma unroll
  for (int s = 0; s < ST - 1; ++s)
    if (s < KT) issue(s, s * BK);

  for (int kt = 0; kt < KT; ++kt) {
    if constexpr (ST >= 3) {
      if (kt + 1 < KT) {
        wait_vmcnt<(ST - 2) * LPT>();
      } else {
        wait_vmcnt<0>();
      }
    } else {
      wait_vmcnt<0>();
    }
    stage_barrier();
    if (kt + ST - 1 < KT) issue((kt + ST - 1) % ST, (kt + ST - 1) * BK);

    // Operand fragments double-buffered across the four 16-deep k-steps: the
    // LDS reads of step kk + 1 are in flight during the MFMAs of step kk.
    const TA* sa = lds + (kt % ST) * T::STAGE;
    V8 af[2][T::TM], wf[2][T::TN];
    auto frags = [&](int kk, int b) {
      const int co = ((2 * kk + g) ^ sw) * 8;
#pragma unroll
      for (int i = 0; i < T::TM; ++i) af[b][i] = *reinterpret_cast<const V8*>(sa + arow + i * 32 * BK + co);
#pragma unroll
      for (int j = 0; j < T::TN; ++j) wf[b][j] = *reinterpret_cast<const V8*>(sa + wrow + j * 32 * BK + co);
    };
    frags(0, 0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      if (kk + 1 < BK / 16) frags(kk + 1, (kk + 1) & 1);
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
#pragma unroll
        for (int i = 0; i < T::TM; ++i) acc[j][i] = mfma32x32x16(wf[kk & 1][j], af[kk & 1][i], acc[j][i]);
    }
  }
}

template <int BM, int BN, int WM, int WN, int ST, int GM, typename TR, typename TC, typename TA>
__global__ __launch_bounds__(WM* WN * 64) void gemm_dma_kernel(const TA* __restrict__ A, const TA* __restrict__ W,
                                                              const float* __restrict__ bias,
                                                              const TR* __restrict__ resid, TC* __restrict__ C,
                                                              int64_t M, int N, int K,
                                                              const uint8_t* __restrict__ row_mask, int epi) {
  using T = DmaTile<BM, BN, WM, WN, ST>;
  constexpr int NT = T::NT;
  __shared__ __attribute__((aligned(1024))) char smem[T::LDS];

  // Tile order: each XCD runs a contiguous range of tile ids; within it, ids
  // walk GM row blocks x all column blocks, so the tiles resident on one XCD
  // at a time share a few A row blocks and W column blocks in its L2.
  const int nbn = (N + BN - 1) / BN;
  const int nbm = (int)((M + BM - 1) / BM);
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int group = tile / (GM * nbn);
  const int first_m = group * GM;
  const int gm = min(nbm - first_m, GM);
  const int in_group = tile - group * GM * nbn;
  const int64_t m0 = (int64_t)(first_m + in_group % gm) * BM;
  const int n0 = (in_group / gm) * BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, g = lane >> 5;

  f32x16 acc[T::TN][T::TM];
  dma_mainloop<BM, BN, WM, WN, ST>(A, W, M, N, K, m0, n0, smem, acc);
  __syncthreads();  // every wave is done with the operand stages

  // Epilogue in TN slices: slice j holds, for every wave column wn, the 32
  // output columns wn*WTN + j*32 .. +31 (EPW = WN * 32 columns in all), staged
  // as fp32 rows (+ bias), then written 16 bytes per lane (CPL columns: 8 fp16 or 4
  // fp32) with the residual added.  Lane li owns row wm*WTM + i*32 + li and, per
  // register quad q, columns 8q + 4g .. 8q + 4g + 3 of its 32-column block.
  float* Cs = reinterpret_cast<float*>(smem);
  constexpr int CPL = 16 / (int)sizeof(TC);  // output columns per lane and store
  constexpr int LPR = T::EPW / CPL;          // lanes per staged row
  constexpr int RPP = NT / LPR;              // rows per pass
  static_assert(NT % LPR == 0 && BM % RPP == 0 && 32 % CPL == 0, "epilogue geometry");
  const int cl = (tid % LPR) * CPL;                               // column within the slice
  const int ccol = (cl / 32) * T::WTN + (cl % 32);                // column within the tile (+ j*32)
#pragma unroll
  for (int j = 0; j < T::TN; ++j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int scol = wn * 32 + 8 * q + 4 * g;
      const int tcol = wn * T::WTN + j * 32 + 8 * q + 4 * g;
      f32x4 bq = {0.f, 0.f, 0.f, 0.f};
      if (bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) bq[e] = n0 + tcol + e < N ? bias[n0 + tcol + e] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < T::TM; ++i) {
        const int row = wm * T::WTM + i * 32 + li;
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[j][i][4 * q + e] + bq[e];
        *reinterpret_cast<f32x4*>(Cs + row * T::LDC + scol) = v;
      }
    }
    __syncthreads();
    const int n = n0 + ccol + j * 32;
    if (n < N) {  // N % 8 == 0, so a lane's CPL columns are all in or all out
      for (int r = tid / LPR; r < BM; r += RPP) {
        const int64_t m = m0 + r;
        if (m >= M) break;
        float v[CPL];
#pragma unroll
        for (int h = 0; h < CPL / 4; ++h) {
          const f32x4 t = *reinterpret_cast<const f32x4*>(Cs + r * T::LDC + cl + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * h + e] = t[e];
        }
        float mv = 1.f;
        if (epi) {
          if (epi & (kEpiMaskBranch | kEpiMaskResid)) mv = row_mask[m] != 0 ? 1.f : 0.f;
          if (epi & kEpiGelu) {
#pragma unroll
            for (int e = 0; e < CPL; ++e) v[e] = gelu_erf(v[e]);
          }
          if ((epi & kEpiMaskBranch) && mv == 0.f) {
#pragma unroll
            for (int e = 0; e < CPL; ++e) v[e] = 0.f;
          }
        }
        if (resid) {
          const TR* rp = resid + m * N + n;
#pragma unroll
          for (int e = 0; e < CPL; ++e) v[e] += to_float(rp[e]);
        }
        if (epi & kEpiMaskResid) {
#pragma unroll
          for (int e = 0; e < CPL; ++e) v[e] *= mv;
        }
        TC* cp = C + m * N + n;
        if constexpr (sizeof(TC) == 4) {
          *reinterpret_cast<f32x4*>(cp) = f32x4{v[0], v[1], v[2], v[3]};
        } else {
          typename Op16<TC>::V8 hv;
#pragma unroll
          for (int e = 0; e < 8; ++e) hv[e] = (TC)v[e];
          *reinterpret_cast<typename Op16<TC>::V8*>(cp) = hv;
        }
      }
    }
    __syncthreads();
  }
}

template <int BM, int BN, int WM, int WN, int ST, int GM, typename TR, typename TC, typename TA>
static hipError_t launch_dma(const GemmArgs& a) {
  const int64_t tiles = ((a.M + BM - 1) / BM) * (int64_t)((a.N + BN - 1) / BN);
  if (tiles > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, WM, WN, ST, GM, TR, TC, TA>), dim3((unsigned)tiles), dim3(WM * WN * 64),
                     0, a.stream, static_cast<const TA*>(a.a), static_cast<const TA*>(a.w), a.bias,
                     static_cast<const TR*>(a.resid), static_cast<TC*>(a.c), a.M, a.N, a.K, a.row_mask, a.epi);
  return hipGetLastError();
}

// Tile choice.  Candidates (measured on MI355X, TFLOP/s at 8192^3 in brackets):
//   256 x 256, 8 waves of 64 x 128   [1096]  one workgroup per CU
//   256 x 192, 8 waves of 64 x 96    [ 980]
//   256 x 128, 8 waves of 64 x 64    [ 951]
//   128 x 128, 4 waves of 64 x 64    [ 932]  two workgroups per CU
// Bigger tiles move fewer bytes through LDS and L2 per MFMA, but a grid that
// ends in a partly filled round wastes CUs.  The estimate below is the number
// of rounds of tiles times the time of one round (tile area / relative
// efficiency); it picks 256 x 192 for 8192 x 3072 x 1024 (2 full rounds; +10 %
// over 128 x 128), 256 x 128 for 8192 x 1024 x 1024 (+6 %) and 256 x 256 for
// the 3.2 M-row projections (+13-16 %).
struct TileCand {
  int bm, bn, per_cu;  // tile and workgroups resident per CU
  double eff;          // relative throughput of a full round
};
constexpr TileCand kTiles[] = {{256, 256, 1, 1.00}, {256, 192, 1, 0.90}, {256, 128, 1, 0.87}, {128, 128, 2, 0.85}};

static int pick_tile(int64_t M, int N) {
  const int64_t cus = compute_units();
  int best = 0;
  double best_t = 1e300;
  for (int i = 0; i < (int)(sizeof(kTiles) / sizeof(kTiles[0])); ++i) {
    const TileCand& c = kTiles[i];
    const int64_t tiles = ((M + c.bm - 1) / c.bm) * (int64_t)((N + c.bn - 1) / c.bn);
    const int64_t slots = cus * c.per_cu;
    const int64_t rounds = (tiles + slots - 1) / slots;
    // a round with more tiles than CUs shares each CU between per_cu workgroups
    const double per_round = (double)c.bm * c.bn / c.eff * (tiles > cus ? c.per_cu : 1);
    const double t = (double)rounds * per_round;
    if (t < best_t * 0.999) {
      best_t = t;
      best = i;
    }
  }
  return best;
}

template <typename TR, typename TC, typename TA = f16>
static hipError_t dispatch_dma(const GemmArgs& a) {
  switch (pick_tile(a.M, a.N)) {
    case 0: return launch_dma<256, 256, 4, 2, 2, 4, TR, TC, TA>(a);
    case 1: return launch_dma<256, 192, 4, 2, 2, 4, TR, TC, TA>(a);
    case 2: return launch_dma<256, 128, 4, 2, 2, 4, TR, TC, TA>(a);
    default: return launch_dma<128, 128, 2, 2, 2, 8, TR, TC, TA>(a);
  }
}

// Out-projection with LayerNorm over whole rows wider than one tile (N = NB * BN; a, W, x
// and y fp16 or bf16): y = LN(x + mask(a W^T + bias)) * gamma + beta, without the branch ever
// reaching memory (the reference's _gemm_kernel + _add_ln_kernel pair for d_model > 128,
// torch_transformer_benchmark.py:1274-1283, 491-535).
//
// The NB column tiles of a BM-row block hold disjoint column ranges of the same rows.
// Each reduces its rows to (mean, M2) over its BN columns (two passes over registers)
// and publishes them as one 64-bit word per row; the row-phase lanes then read the
// words of all NB tiles, polling until none holds the "not yet written" pattern the
// preceding kernel of the sublayer filled the area with, and combine them exactly (Chan
// et al.: mean of the tile means, M2 = sum M2_t + BN sum (mean_t - mean)^2).  The words
// move through agent-scope atomics (stores and loads at the device coherence point,
// past the XCD-local L2s); a 64-bit word is written whole, so a reader sees either the
// fill pattern or the published statistics, and needs no fence, counter or barrier.
//
// Co-residency: the launcher runs this kernel only when the whole grid fits the chip
// at one workgroup per CU.  Tile ids are dealt to XCDs in contiguous ranges
// (xcd_remap) and a row block's tiles are consecutive ids, so every XCD dispatches all
// of a row block's tiles before any tile of a later row block: the tiles a waiting tile
// depends on are never queued behind tiles that wait on it, and with fewer CUs free the
// row blocks still complete in order.  The wait is bounded all the same (spin_limit
// polls); a wave that gives up writes NaN rows rather than hanging.  Each wave reads the
// words of its own rows only, so no barrier follows the publication.
template <int BM, int BN, int WM, int WN, int ST, int NB, bool MASKED, typename TA>
__global__ __launch_bounds__(WM* WN * 64) void gemm_dma_rowln_kernel(
    const TA* __restrict__ A, const TA* __restrict__ W, const float* __restrict__ bias, const TA* __restrict__ x,
    const float* __restrict__ gamma, const float* __restrict__ beta, TA* __restrict__ y, int64_t M, int K,
    float eps, const uint8_t* __restrict__ row_mask, uint64_t* __restrict__ stats, int spin_limit) {
  using T = DmaTile<BM, BN, WM, WN, ST>;
  constexpr int NT = T::NT, N = NB * BN;
  constexpr int LDC = BN + 4;          // fp32 staging row stride (floats)
  constexpr int LPR = BN / 8;          // lanes per row in the row phase, 8 columns each
  constexpr int RPP = NT / LPR;        // rows per pass
  constexpr int NP = BM / RPP;         // passes
  constexpr int LDSB = T::LDS > BM * LDC * 4 ? T::LDS : BM * LDC * 4;
  static_assert(NB >= 2 && NB <= LPR && (NB & (NB - 1)) == 0, "one tile's statistics per lane of a row group");
  static_assert(NT % LPR == 0 && BM % RPP == 0 && LDSB <= 163840, "row-phase geometry");
  __shared__ __attribute__((aligned(1024))) char smem[LDSB];

  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int rb = tile / NB, tc = tile % NB;
  const int64_t m0 = (int64_t)rb * BM;
  const int n0 = tc * BN;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 31, g = lane >> 5;
  const int cl = (tid % LPR) * 8;  // row phase: this lane's 8 columns of the tile
  const int rl = tid / LPR;        // and its row within each pass

  // Everything the epilogue reads from memory is requested before the k-loop: the
  // residual rows of the row phase, the bias of this lane's accumulator columns, the
  // row-mask bytes, gamma and beta.  The first k-tile waits for all transfers in flight
  // anyway (its LDS-DMA), so these cost one round trip there and none later (issued
  // inside the loop, the LDS reads after them would wait for them).
  typename Op16<TA>::V8 xr[NP];
  f32x4 bq[T::TN][4];
  uint8_t mb[T::TM];
  f32x4 gv4[2], bv4[2];
  {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int64_t m = min(m0 + p * RPP + rl, M - 1);
      xr[p] = *reinterpret_cast<const typename Op16<TA>::V8*>(x + m * N + n0 + cl);
    }
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        bq[j][q] = *reinterpret_cast<const f32x4*>(bias + n0 + wn * T::WTN + j * 32 + 8 * q + 4 * g);
    if constexpr (MASKED) {
#pragma unroll
      for (int i = 0; i < T::TM; ++i) mb[i] = row_mask[min(m0 + wm * T::WTM + i * 32 + li, M - 1)];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      gv4[h] = *reinterpret_cast<const f32x4*>(gamma + n0 + cl + 4 * h);
      bv4[h] = *reinterpret_cast<const f32x4*>(beta + n0 + cl + 4 * h);
    }
  }
  f32x16 acc[T::TN][T::TM];
  dma_mainloop<BM, BN, WM, WN, ST>(A, W, M, N, K, m0, n0, smem, acc);
  __syncthreads();  // every wave is done with the operand stages

  // Branch a W^T + bias, zero on padded rows, staged as fp32 rows of the tile.
  float* Cs = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int j = 0; j < T::TN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = wn * T::WTN + j * 32 + 8 * q + 4 * g;
#pragma unroll
      for (int i = 0; i < T::TM; ++i) {
        const int row = wm * T::WTM + i * 32 + li;
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[j][i][4 * q + e] + bq[j][q][e];
        if constexpr (MASKED) {
          if (mb[i] == 0) v = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        *reinterpret_cast<f32x4*>(Cs + row * LDC + col) = v;
      }
    }
  __syncthreads();

  // r = x + branch; per row of the tile, LPR lanes hold 8 columns each: the tile's
  // mean, then M2 around it, published as one 64-bit word per row.
  float r[NP][8];
  uint64_t* my_stats = stats + ((int64_t)rb * NB + tc) * BM;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row = p * RPP + rl;
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(Cs + row * LDC + cl);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(Cs + row * LDC + cl + 4);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      r[p][e] = (float)xr[p][e] + (e < 4 ? c0[e] : c1[e - 4]);
      s += r[p][e];
    }
    const float mean_t = group_sum<LPR>(s) * (1.0f / BN);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = r[p][e] - mean_t;
      q += d * d;
    }
    q = group_sum<LPR>(q);
    if (tid % LPR == 0) {
      const uint64_t word = (uint64_t)__float_as_uint(mean_t) | ((uint64_t)__float_as_uint(q) << 32);
      __hip_atomic_store(my_stats + row, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // Lane j of a row group reads tile j % NB's word of each of its rows, until none is
  // the fill pattern (the wave polls as one); each aligned group of NB lanes then holds
  // every tile once.
  const uint64_t* row_stats = stats + ((int64_t)rb * NB + (tid % LPR) % NB) * BM + rl;
  uint64_t w[NP];
  bool ok = true;
  for (int polls = 0;; ++polls) {
    bool pending = false;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      w[p] = __hip_atomic_load(row_stats + p * RPP, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pending = pending || w[p] == kRowLnUnset;
    }
    if (!__builtin_amdgcn_ballot_w64(pending)) break;
    if (polls >= spin_limit) {
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }

  float gv[8], bv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    gv[e] = gv4[e >> 2][e & 3];
    bv[e] = bv4[e >> 2][e & 3];
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const float mean_t = __uint_as_float((uint32_t)w[p]);
    const float m2_t = __uint_as_float((uint32_t)(w[p] >> 32));
    const float mean = group_sum<NB>(mean_t) * (1.0f / NB);
    const float d = mean_t - mean;
    const float m2 = group_sum<NB>(m2_t + (float)BN * d * d);
    const float rstd = ok ? rsqrtf(m2 * (1.0f / N) + eps) : __builtin_nanf("");
    const int64_t m = m0 + p * RPP + rl;
    if (m < M) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (r[p][e] - mean) * rstd * gv[e] + bv[e];
      store8(y + m * N + n0 + cl, o);
    }
  }
}

template <int NB, bool MASKED, typename TA>
static hipError_t launch_rowln(const GemmRowLnArgs& a) {
  constexpr int BM = 256, BN = 128;
  const int64_t nbm = (a.M + BM - 1) / BM;
  hipLaunchKernelGGL((gemm_dma_rowln_kernel<BM, BN, 4, 2, 2, NB, MASKED, TA>), dim3((unsigned)(nbm * NB)), dim3(512),
                     0, a.stream, static_cast<const TA*>(a.a), static_cast<const TA*>(a.w), a.bias,
                     static_cast<const TA*>(a.x), a.gamma, a.beta, static_cast<TA*>(a.y), a.M, a.K, a.eps,
                     a.row_mask, static_cast<uint64_t*>(a.sync), 1 << 20);
  return hipGetLastError();
}

template <int NB>
static hipError_t launch_rowln(const GemmRowLnArgs& a) {
  if (a.dtype == kBF16)
    return a.row_mask ? launch_rowln<NB, true, bf16>(a) : launch_rowln<NB, false, bf16>(a);
  return a.row_mask ? launch_rowln<NB, true, f16>(a) : launch_rowln<NB, false, f16>(a);
}

bool gemm_rowln_ok(int64_t M, int N, int K) {
  // 128-wide column tiles, 2 .. 16 per row; K in whole k-tiles with 32-bit block offsets;
  // the whole grid resident at once (one 256 x 128 tile per CU).
  if (M <= 0 || K <= 0 || K % 64 != 0 || (int64_t)256 * K * 2 >= ((int64_t)1 << 32)) return false;
  if (N != 256 && N != 512 && N != 1024 && N != 2048) return false;
  const int64_t tiles = ((M + 255) / 256) * (N / 128), cus = compute_units();
  // Worth it once the grid covers most of the chip: the GEMM + LayerNorm pass it replaces
  // spreads smaller tiles over every CU.  Measured in-graph at d_model 1024 against that
  // pair: 64 tiles +5.1 us, 128 +2.6, 192 -0.5, 256 -2.5; at d_model 512 (K = 512) 128
  // tiles -4.1 us.
  return tiles <= cus && (4 * tiles >= 3 * cus || (K <= 512 && 2 * tiles >= cus));
}

int64_t gemm_rowln_sync_bytes(int64_t M, int N) { return (M + 255) / 256 * (N / 128) * 256 * 8; }

hipError_t run_gemm_rowln(const GemmRowLnArgs& a) {
  if (!a.a || !a.w || !a.bias || !a.x || !a.gamma || !a.beta || !a.y || !a.sync || !gemm_rowln_ok(a.M, a.N, a.K))
    return hipErrorInvalidValue;
  if (a.dtype != kF16 && a.dtype != kBF16) return hipErrorInvalidValue;
  switch (a.N / 128) {
    case 2: return launch_rowln<2>(a);
    case 4: return launch_rowln<4>(a);
    case 8: return launch_rowln<8>(a);
    default: return launch_rowln<16>(a);
  }
}

bool gemm_dma_ok(const GemmArgs& a) {
  // K in whole 64-wide k-tiles; N in 8-column groups; a per-block byte offset
  // (rows x K) that fits 32 bits; at least half a round of 128 x 128 tiles.
  if (a.ln_gamma || a.K % 64 != 0 || a.N % 8 != 0 || a.M <= 0) return false;
  if ((int64_t)256 * a.K * 2 >= ((int64_t)1 << 32)) return false;
  const int64_t tiles = ((a.M + 127) / 128) * (int64_t)((a.N + 127) / 128);
  return 2 * tiles >= compute_units();
}

hipError_t run_gemm_dma(const GemmArgs& a) {
  if (a.ab_dtype == kBF16) {  // residual bf16 or fp32, output bf16 or fp32
    const bool rb = !a.resid || a.resid_dtype == kBF16;
    if (a.c_dtype == kBF16) return rb ? dispatch_dma<bf16, bf16, bf16>(a) : dispatch_dma<float, bf16, bf16>(a);
    return rb ? dispatch_dma<bf16, float, bf16>(a) : dispatch_dma<float, float, bf16>(a);
  }
  const bool c16 = a.c_dtype == kF16;
  if (!a.resid || a.resid_dtype == kF16) return c16 ? dispatch_dma<f16, f16>(a) : dispatch_dma<f16, float>(a);
  return c16 ? dispatch_dma<float, f16>(a) : dispatch_dma<float, float>(a);
}

}  // namespace cobra
