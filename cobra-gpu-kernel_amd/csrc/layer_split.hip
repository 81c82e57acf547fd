// The whole attention sublayer in one kernel, split by query slices so that a
// small batch still covers the chip: workgroup (b, s) produces the outputs of
// queries 32s .. 32s+31 of sequence b (S <= 128, fp16 activations, d_model
// 64 or 128, head_dim 32 or 64).
//
//   h = LN1(x);  q,k,v = h W^T + b;  ctx = softmax(q k^T * scale) v;
//   r = x + ctx W_o^T + b_o;  y = LN2(r)
//
// Same fusion of the reference's _add_ln_kernel, _qkvattn_kernel and
// _gemm_ln_kernel (torch_transformer_benchmark.py:491-535, 654-741, 394-463)
// and the same fragment conventions as the persistent kernel; what changes is
// the division of work.  The persistent kernel gives one workgroup a whole
// sequence and walks the heads one after another; here the S/32 workgroups of a
// sequence run side by side, and inside a workgroup the waves split every
// phase four ways:
//   1. wave w normalises tokens 32w .. 32w+31 (LN1, mean and variance in one
//      pass) while the W_k / W_v rows of d-tile w arrive; the wave whose tile
//      holds the slice's own queries keeps a raw copy of it, the residual;
//   2. wave w projects K^T and V of d-tile w for ALL tokens (every workgroup
//      of the sequence recomputes them: twice the projection FLOPs of the
//      persistent kernel, but no cross-workgroup traffic at all), and Q^T of
//      the slice for head w;
//   3. wave h runs the attention of head h over all keys; the softmax is
//      exact, every key of the sequence is present.  With one head of 128
//      dims the waves split it instead: wave w projects Q^T d-tile w, scores
//      key tile w, the row max / sum and the probabilities go through LDS,
//      and wave w forms output d-tile w over all keys.  With 8-dim heads
//      wave w takes the four heads of d-tile w (each 16-dim k-step holds two
//      heads: the other head's half of the K fragment is zeroed);
//   4. wave n multiplies the gathered attention output by the W_o rows of
//      output columns 32n .. 32n+31, adds bias and residual, and LN2 combines
//      the per-wave row sums and sums of squares through LDS in one exchange.
//
// Every global read is an LDS-DMA (global_load_lds_dwordx4) of whole 1 KB
// spans: matrix rows land row-major in LDS with 16-byte chunks XOR-swizzled by
// row, and each lane then reads its MFMA operand fragment (row = lane % 32) from
// there without bank conflicts.  Reading operands straight from global memory
// in that layout would touch 32 rows per load instruction; the coalesced DMA
// moves the same bytes several times faster.  A wave only ever reads what its
// own DMA wrote until the first barrier, so it waits for exactly the
// transfers it needs (vmcnt retires in issue order); the barriers publish LDS
// writes without waiting for DMA still in flight.
#include "common.hpp"
#include "kernels.hpp"
#include "layer_common.hpp"
#include "lds_dma.hpp"

namespace cobra {

namespace {

constexpr int kSplitWaves = 4;
constexpr int kSplitTiles = kSmallMaxS / 32;  // token tiles of a sequence

// LDS plan (bytes) and per-wave DMA counts; BLK: the whole-block mode.
template <int D, int HD, bool BLK>
struct SplitPlan {
  static constexpr int KD = D / 16;    // k-steps over d_model
  static constexpr int NNT = D / 32;   // 32-wide tiles of d_model
  static constexpr int H = D / HD;
  static constexpr int NDT = HD / 32;  // 32-wide d tiles per head
  static constexpr int KSH = HD / 16;  // k-steps per head
  // One head wider than a wave's share (head_dim 128): Q^T and the attention are
  // split across the waves by d-tile / key tile rather than given to wave 0.
  static constexpr bool QSPLIT = HD > 64;
  // Heads narrower than a k-step (head_dim 8): wave w owns the four heads of d-tile w.
  static constexpr bool NARROW = HD < 16;
  // Q^T is projected by d-tile (wave w: rows 32w .. 32w+31 of W_q) rather than by head.
  static constexpr bool QBYTILE = QSPLIT || NARROW;
  static constexpr int NQT = QBYTILE ? 1 : NDT;  // Q^T d-tiles one wave projects
  static constexpr int ROWB = 2 * D;                   // one fp16 row of d_model
  static constexpr int TILEB = 32 * ROWB;              // 32 such rows
  static constexpr int KVB = 2 * kSplitTiles * KD * 1024;  // K^T then V fragments (1 KB each)
  static constexpr int WKVB = NNT * 2 * TILEB;         // W_k / W_v rows, staged per d-tile
  static constexpr int A = KVB > WKVB ? KVB : WKVB;    // W_k/W_v staging, then K^T / V
  static constexpr int X = kSplitWaves * TILEB;        // token tiles, then LN1 output fragments
  static constexpr int Q = D * ROWB;                   // W_q rows, then W_o rows
  static constexpr int CX = KD * 1024;                 // attention output fragments
  // The residual of the slice: raw fp16 fragments of its token tile, or (whole-block
  // mode) the fp32 rows of the block's residual, 4 KB per wave.
  static constexpr int RAWB = BLK ? kSplitWaves * 4096 : KD * 1024;
  // Parameter rows of one wave, then [gamma1 | beta1] (or, whole-block mode, b1 | b2 | the next norm).
  static constexpr int PB = BLK ? 1536 : 2048;
  static constexpr int OFF_X = A, OFF_Q = OFF_X + X, OFF_CX = OFF_Q + Q, OFF_R = OFF_CX + CX;
  static constexpr int OFF_P = OFF_R + RAWB, OFF_STAT = OFF_P + kSplitWaves * PB;
  static constexpr int BYTES = OFF_STAT + 2 * kSplitWaves * 32 * 4;
  // DMA instructions of one wave, in issue order: [gamma1|beta1] 1 (affine LN1 only),
  // token tile N_X, other parameters 1, W_k/W_v N_A before barrier 1; W_q N_Q between
  // the first token tiles' K / V products; W_o N_O after barrier 2.
  static constexpr int N_X = TILEB / 1024, N_A = 2 * TILEB / 1024, N_Q = NQT * TILEB / 1024;
  static constexpr int N_O = TILEB / 1024;
  static_assert(D == 64 || D == 128, "swizzle and row geometry");
  static_assert((HD == 8 || HD == 32 || HD == 64 || HD == 128) && D % HD == 0, "head geometry");
  static_assert(!QSPLIT || (H == 1 && NDT == kSplitWaves), "a split head has one d / key tile per wave");
  static_assert(!NARROW || (D == 128 && NNT == kSplitWaves), "narrow heads: four per wave, one d-tile per wave");
  static_assert((NARROW || H <= kSplitWaves) && NNT <= kSplitWaves, "one wave per head and per d / output tile");
  static_assert(KD * 1024 == TILEB, "LN1 output fragments of a tile fill its input tile");
  static_assert(!QSPLIT || KSH * 1024 == CX, "the split head's Q^T fragments fit the attention-output area");
  static_assert(2 * D * 4 <= 1024 && 2 * 32 + NQT * 32 + 3 * 32 <= 256, "parameter rows");
  static_assert(1 + N_X + 1 + N_A + N_Q < 64, "vmcnt range");
  static_assert(BYTES <= kLdsBytes, "LDS budget");
};

// 16-byte chunk c of row r of a row-major fp16 tile with D columns sits at
// chunk c ^ swz(r): 16 consecutive rows read at one chunk hit 16 distinct
// 4-bank groups.
template <int D>
__device__ __forceinline__ int row_swz(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}

// DMA of `NI` 1 KB spans of a swizzled row-major [rows][D] fp16 tile at `dst`;
// src_row(r) is the global address of tile row r.
template <int D, int NI, typename F>
__device__ __forceinline__ void dma_rows(char* dst, int lane, F src_row) {
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int o = 1024 * i + 16 * lane;
    const int r = o / (2 * D), pos = (o % (2 * D)) / 16;
    dma16(src_row(r) + 8 * (pos ^ row_swz<D>(r)), dst + 1024 * i);
  }
}

// The same transfer for a tile whose rows are contiguous in memory (row r at
// base + r * 2D bytes, `base` wave-uniform).  Instruction i moves, per lane, the
// 16 bytes at base + 1024 i + off[i % NP]: the swizzle repeats every NP spans,
// so the per-lane part is NP registers computed once, the rest is a scalar base
// plus an immediate (no 64-bit per-lane address arithmetic per transfer).
template <int D>
struct RowSpans {
  static constexpr int NP = D == 128 ? 4 : 2;
  uint32_t off[NP];
  __device__ __forceinline__ explicit RowSpans(int lane) {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int o = 1024 * j + 16 * lane;
      const int r = o / (2 * D), pos = (o % (2 * D)) / 16;
      off[j] = (uint32_t)(r * 2 * D - 1024 * j + 16 * (pos ^ row_swz<D>(r)));
    }
  }
};

template <int D, int NI>
__device__ __forceinline__ void dma_span_rows(char* dst, const char* base, const RowSpans<D>& sp) {
#pragma unroll
  for (int i = 0; i < NI; ++i) dma16(base + 1024 * i + sp.off[i % RowSpans<D>::NP], dst + 1024 * i);
}

// Operand fragment of tile row r, logical chunk c.
template <int D>
__device__ __forceinline__ f16x8 tile_chunk(const char* tile, int r, int c) {
  return *reinterpret_cast<const f16x8*>(tile + r * 2 * D + 16 * (c ^ row_swz<D>(r)));
}

}  // namespace

// The rest of a transformer block, for the whole-block mode of the kernel: the
// input is then h = norm1(r) (fp16) and the residual r comes from `rin` (fp32).
struct BlockTail {
  const float* rin;   // [B*S, D] residual entering the block (may equal the kernel's resid_out)
  const f16* w1;      // [F, D] ffn_in weight
  const float* b1;    // [F]
  const f16* w2;      // [D, F] ffn_out weight
  const float* b2;    // [D]
  const float* gn;    // the next norm (next block's norm1, or final_norm)
  const float* bn;
  int y_f32;          // output dtype: fp32 if set, else fp16
  int mask_out;       // multiply the normalised output of padded rows by 0
};

// The whole-block mode adds the rest of the block.
template <bool BLK>
struct SplitKArgs : SplitArgs {};
template <>
struct SplitKArgs<true> : SplitArgs {
  BlockTail tail;
};

// AFF1: LN1 with an elementwise affine (g1 / be1 non-null; never in whole-block mode).
//
// The first eight arguments repeat fields of `ka` as scalars: the ones the first
// transfers need.  Built with -amdgpu-kernarg-preload-count, they arrive in SGPRs
// when the wave starts (gfx950 kernel-argument preloading), so the token tile and the
// parameter segments are requested without waiting for the kernel-argument loads;
// the rest of `ka` loads meanwhile.
template <int D, int HD, bool CAUSAL, bool MASKED, bool BLK, bool AFF1>
__global__ __launch_bounds__(64 * kSplitWaves) void layer_split_kernel(int S_, int nblk_, const f16* x_, const f16* wqkv_,
                                                                     const float* bqkv_, const float* bo_,
                                                                     const float* g2_, const float* be2_,
                                                                     const SplitKArgs<BLK> ka) {
  const int S = S_, nblk = nblk_;
  const f16* __restrict__ x = x_;
  const f16* __restrict__ wqkv = wqkv_;
  const float* __restrict__ bqkv = bqkv_;
  const float* __restrict__ bo = bo_;
  const float* __restrict__ g2 = g2_;
  const float* __restrict__ be2 = be2_;
  const f16* __restrict__ wo = ka.wo;
  const float* __restrict__ g1 = ka.g1;
  const float* __restrict__ be1 = ka.be1;
  void* __restrict__ yv = ka.y;
  float* resid_out = ka.resid_out;
  const float c2 = ka.c2, eps = ka.eps;
  const uint8_t* __restrict__ vmask = ka.vmask;
  const BlockTail tail = [&] {
    if constexpr (BLK)
      return ka.tail;
    else
      return BlockTail{};
  }();
  using P = SplitPlan<D, HD, BLK>;
  constexpr int KD = P::KD, NNT = P::NNT, H = P::H, NDT = P::NDT, KSH = P::KSH, NQT = P::NQT;
  // Whole-block mode: the FFN's hidden width equals d_model, one 32-wide tile per wave.
  static_assert(!BLK || NNT == kSplitWaves, "whole-block mode: d_model 128");
  f16* const y = static_cast<f16*>(yv);

  __shared__ __attribute__((aligned(1024))) char smem[P::BYTES];
  char* const rA = smem;               // W_k/W_v staging, then K^T | V fragments
  char* const rX = smem + P::OFF_X;    // token tiles, then LN1 output fragments
  char* const rQ = smem + P::OFF_Q;    // W_q rows, then W_o rows
  f16x8* const Kl = reinterpret_cast<f16x8*>(rA);
  f16x8* const Vl = Kl + kSplitTiles * KD * 64;
  f16x8* const Hb = reinterpret_cast<f16x8*>(rX);
  f16x8* const Cx = reinterpret_cast<f16x8*>(smem + P::OFF_CX);
  f16x8* const Qx = Cx;  // split head: Q^T fragments of the slice, read before any Cx store
  f16x8* const Px = Hb;  // split head: probability fragments, once every projection has read Hb
  f16x8* const Raw = reinterpret_cast<f16x8*>(smem + P::OFF_R);  // x rows of the slice, unnormalised
  float* const Stat = reinterpret_cast<float*>(smem + P::OFF_STAT);

  // The S/32 slices of a sequence run on one XCD, so its L2 serves the token
  // tiles they all read.
  const int NS = (S + 31) >> 5;  // query slices per sequence: 1-4 (S <= 128)
  const int item = xcd_remap(blockIdx.x, nblk);
  // item / NS by a shift or, for 3, a multiply (exact for every 32-bit item): the
  // division's reciprocal sequence sat on the path to the first transfer.
  const int b = NS == 3 ? (int)(((uint64_t)(uint32_t)item * 0xAAAAAAABull) >> 33) : item >> (NS >> 1);
  const int s = item - b * NS;  // query slice
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31, g = lane >> 5;
  const int qtok = 32 * s + li;  // query of this lane for attention, out-projection, LN2
  const bool q_ok = qtok < S;
  const f16* xs = x + (int64_t)b * S * D;
  // Waves past the last d-tile / head issue the same transfers for tile / head 0
  // (identical bytes to the same place), so every wave's wait counts are equal.
  const int dq = w < NNT ? w : 0, hq = w < H ? w : 0;
  char* const rP = smem + P::OFF_P + w * P::PB;  // the 32-float parameter segments, then [gamma1 | beta1]
  char* const rWkv = rA + dq * 2 * P::TILEB;
  // W_q rows this wave projects: d-tile dq of the split head, else all of head hq.
  const int qrow0 = P::QBYTILE ? 32 * dq : HD * hq;
  char* const rWq = rQ + (P::QBYTILE ? dq : hq * NDT) * P::TILEB;
  char* const rWo = rQ + dq * P::TILEB;
  char* const rTok = rX + w * P::TILEB;

  // Token mask bytes first: the oldest transfers, so every later vmcnt wait covers them.
  KeyBytes kbytes{1, 1};
  if constexpr (MASKED) {
    kbytes = load_key_bytes(vmask + (int64_t)b * S, S, lane);
    asm volatile("" ::: "memory");
  }

  // ---- DMA, in the order the data is needed -------------------------------------------
  const RowSpans<D> spans(lane);
  static_assert(!(BLK && AFF1), "the whole-block input is already normalised");
  constexpr bool aff1 = AFF1;
  if constexpr (BLK) {  // b1, b2 and the next norm's parameters of tile w (512 bytes: lanes 0-31)
    const int seg = lane >> 3, off = 32 * w + 4 * (lane & 7);
    const float* src = seg == 0 ? tail.b1 + off : seg == 1 ? tail.b2 + off : seg == 2 ? tail.gn + off : tail.bn + off;
    if (lane < 32) dma16(src, rP + 1024);
  } else if (aff1) {  // [gamma1 | beta1] (later vmcnt waits count only what follows the token tile)
    const int c = 4 * lane;
    dma16(c < D ? g1 + c : be1 + (c < 2 * D ? c - D : 0), rP + 1024);
  }
  // Token tile w.  Rows past S fetch row 0 (S >= 1): finite values whose keys the
  // softmax masks and whose queries are never stored.
  if (32 * w + 32 <= S)
    dma_span_rows<D, P::N_X>(rTok, reinterpret_cast<const char*>(xs + (int64_t)32 * w * D), spans);
  else
    dma_rows<D, P::N_X>(rTok, lane, [&](int r) { return xs + (int64_t)(32 * w + r < S ? 32 * w + r : 0) * D; });
  {  // 32-float segments: b_k, b_v of d-tile dq; b_q of the projected Q rows (2 x 32); b_o, gamma2, beta2 of tile dq
    const int seg = lane >> 3, off = 4 * (lane & 7);
    const float* src = seg == 0   ? bqkv + D + 32 * dq + off
                       : seg == 1 ? bqkv + 2 * D + 32 * dq + off
                       : seg == 2 ? bqkv + qrow0 + off
                       : seg == 3 ? bqkv + qrow0 + (NQT > 1 ? 32 : 0) + off
                       : seg == 4 ? bo + 32 * dq + off
                       : seg == 5 ? g2 + 32 * dq + off
                       : seg == 6 ? be2 + 32 * dq + off
                                  : bo + off;
    dma16(src, rP);
  }
  // The W_k and then the W_v rows of d-tile dq are issued from inside LN1, spread
  // evenly over its arithmetic steps, so that LN1 starts as soon as the token tile is in.
  // The CU's load path drains about one 1 KB transfer per 20 cycles; a wave that
  // issues more than the queue holds stalls at the issue, so transfers issued in one
  // run ahead of LN1 would hold LN1 back until the load path had worked through them
  // all.  Only what the K / V products need is loaded before the first barrier: the
  // W_q rows follow between the first token tiles' products and the W_o rows during
  // the attention, so neither is waited for before the matrix cores start.
  const char* const wbytes = reinterpret_cast<const char*>(wqkv);
  constexpr int NV = P::N_A / 2, NKV = 2 * NV, NSLOT = 2 * KD;
  const char* const wksrc = wbytes + (int64_t)(D + 32 * dq) * 2 * D;  // W_k rows, then W_v rows (D rows on)
  const char* const wqsrc = wbytes + (int64_t)qrow0 * 2 * D;
  auto issue_late = [&](int slot) {  // slot < NSLOT: spans ceil(slot NKV / NSLOT) ..
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = (slot * NKV + NSLOT - 1) / NSLOT; j < ((slot + 1) * NKV + NSLOT - 1) / NSLOT; ++j) {
      const int jj = j < NV ? j : j - NV;
      const char* const src = j < NV ? wksrc : wksrc + (int64_t)D * 2 * D;
      dma16(src + 1024 * jj + spans.off[jj % RowSpans<D>::NP], rWkv + (j < NV ? 0 : P::TILEB) + 1024 * jj);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- LN1 of token 32w + li (columns 16kk + 8g + e): its tile is in. ------------------
  KeyBits kbits{~0ull, ~0ull};
  if constexpr (BLK) {
    // The input is already normalised: the projections read the token tiles as they landed.
#pragma unroll
    for (int slot = 0; slot < NSLOT; ++slot) issue_late(slot);
  } else {
  wait_vmcnt<1>();  // the token tile (the parameter segments may be in flight)
  if constexpr (MASKED) kbits = key_bits_of(kbytes, S, lane);
  {
    f16x8 xc[KD];
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) xc[kk] = tile_chunk<D>(rTok, li, 2 * kk + g);
    // The residual rows of the slice, before the tile is overwritten.
    if (w == s) {
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) Raw[kk * 64 + lane] = xc[kk];
    }
    const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
    if (!aff1) {
      // One pass over the tile, shifted by a pilot value p (one element of the row, the
      // same in both lanes of the pair): sums of d = x - p and d^2 by fp16 pair dot
      // products (exact products, fp32 accumulation, independent chains), variance
      // E[d^2] - E[d]^2.  The shift keeps that difference well conditioned when the
      // row's mean is large against its spread (E[x^2] - mean^2 loses every digit at a
      // mean of ~1000 standard deviations); d is rounded to fp16 once, relative to |d|.
      // Then h = x rstd - mean rstd, a mixed-precision fma per element (fp16 x, fp32
      // arithmetic) and one rounding to fp16.
      const f16 pil = pair_pilot(xc[0][0]);
      const f16x2 p2 = {pil, pil};
      float s1[2] = {0.f, 0.f}, s2[2] = {0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 pr = pk_sub_f16(f16x2{xc[kk][2 * e], xc[kk][2 * e + 1]}, p2);
          s1[e & 1] = __builtin_amdgcn_fdot2(pr, one2, s1[e & 1], false);
          s2[e & 1] = __builtin_amdgcn_fdot2(pr, pr, s2[e & 1], false);
        }
        issue_late(kk);
      }
      const float md = sum_xor32(s1[0] + s1[1]) * (1.0f / D);
      const float ed2 = sum_xor32(s2[0] + s2[1]) * (1.0f / D);
      const float rstd = rsqrtf(fmaxf(ed2 - md * md, 0.f) + eps);
      const float mean = (float)pil + md;
      const float nmr = -mean * rstd;
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) {
        f16x8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (f16)fmaf((float)xc[kk][e], rstd, nmr);
        Hb[(w * KD + kk) * 64 + lane] = h;
        issue_late(KD + kk);
      }
    } else {
#pragma unroll
      for (int slot = 0; slot < NSLOT; ++slot) issue_late(slot);
      float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KD; ++kk)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          part[e] = __builtin_amdgcn_fdot2(f16x2{xc[kk][2 * e], xc[kk][2 * e + 1]}, one2, part[e], false);
      const float mean = sum_xor32((part[0] + part[1]) + (part[2] + part[3])) * (1.0f / D);
      const float* pg = reinterpret_cast<const float*>(rP + 1024);
      float gv[KD][8], bv[KD][8];
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) {
        load8(pg + 16 * kk + 8 * g, gv[kk]);
        load8(pg + D + 16 * kk + 8 * g, bv[kk]);
      }
      float xv[KD][8];
      float qp[2] = {0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KD; ++kk)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xv[kk][e] = (float)xc[kk][e] - mean;
          qp[e & 1] = fmaf(xv[kk][e], xv[kk][e], qp[e & 1]);
        }
      const float r1 = rsqrtf(sum_xor32(qp[0] + qp[1]) * (1.0f / D) + eps);
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) {
        f16x8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (f16)fmaf(xv[kk][e] * r1, gv[kk][e], bv[kk][e]);
        Hb[(w * KD + kk) * 64 + lane] = h;
      }
    }
    // (The fragments overwrite the token tile in place: every read of it above
    // precedes the first write.)
  }
  }

  // ---- operand fragments of this wave's weights -------------------------------------------
  wait_vmcnt<0>();
  if constexpr (BLK && MASKED) kbits = key_bits_of(kbytes, S, lane);  // the mask bytes are older
  f16x8 wk[KD], wv[KD];  // A operand of K^T = W_k h^T; B operand of V = h W_v^T
#pragma unroll
  for (int kk = 0; kk < KD; ++kk) {
    wk[kk] = tile_chunk<D>(rWkv, li, 2 * kk + g);
    wv[kk] = tile_chunk<D>(rWkv + P::TILEB, li, 2 * kk + g);
  }
  const float* pp = reinterpret_cast<const float*>(rP);  // the 32-float segments above
  // The barrier that publishes every wave's LN1 output comes after this wave's products
  // on its own token tile (below): that tile is its own LN1 output (or its own DMA in
  // the whole-block mode), and the other waves finish their LN1 meanwhile.

  // Whole-block mode: the residual entering the block, rows of the slice x columns
  // 32w .. 32w+31 (fp32, 128 bytes a row), into this wave's 4 KB of the residual area,
  // before any later transfer so the wait for the W_o rows covers it.  16-byte chunk c of
  // row r sits at chunk c ^ (r & 7): the epilogue's reads (32 rows, one chunk) are then
  // conflict-free.  (Held in registers instead, the rows were moved to spill registers
  // as soon as they were requested, a wait for every transfer in flight.)  Rows past S
  // read row 0 of the sequence (unused).
  char* const rRes = smem + P::OFF_R + w * 4096;
  if constexpr (BLK) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 8 * i + (lane >> 3), c = (lane & 7) ^ (r & 7);
      const int tok = 32 * s + r < S ? 32 * s + r : 0;
      dma16(tail.rin + ((int64_t)b * S + tok) * D + 32 * w + 4 * c, rRes + 1024 * i);
    }
  }

  // W_q rows qrow0 .. qrow0 + 32 NQT - 1 of a wave that projects Q^T, issued at the
  // start of the first token tiles' products (the matrix cores are busy with those
  // while the wave waits at the issue) and read back at the last tile.
  const bool doq = P::QBYTILE || w < H;
  constexpr int kWqPer = (P::N_Q + kSplitTiles - 2) / (kSplitTiles - 1);  // spans per tile 0 ..
  auto issue_wq = [&](int t) {  // t < kSplitTiles - 1
#pragma unroll
    for (int i = t * kWqPer; i < (t + 1) * kWqPer && i < P::N_Q; ++i)
      dma16(wqsrc + 1024 * i + spans.off[i % RowSpans<D>::NP], rWq + 1024 * i);
  };
  f16x8 wq[NQT][KD];  // A operand of Q^T = W_q h^T

  // ---- K^T and V of d-tile w for every token tile; Q^T of the slice for head w ---------
  f16x8 qB[P::NARROW ? 2 : KSH];  // B operand of S^T = K Q^T (narrow heads: the two k-steps of d-tile w)
  if (w < NNT) {
    // The biases start the accumulators (the first product of each chain reads them
    // as its C operand), so no bias add follows the products.
    f32x16 bk, bv;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(pp + 8 * qd + 4 * g);
#pragma unroll
      for (int e = 0; e < 4; ++e) bk[4 * qd + e] = t[e];
    }
    const float bvl = pp[32 + li];
#pragma unroll
    for (int r = 0; r < 16; ++r) bv[r] = bvl;
    // Head and d tile within the head (head-major K / V areas); narrow heads keep
    // K^T by 16-dim k-step of d_model and V by d-tile instead.
    const int h = P::NARROW ? 0 : (32 * w) / HD, t2 = P::NARROW ? 0 : w % (P::NARROW ? 1 : NDT);
    // Two accumulator pairs: the products of token tile t run on the matrix
    // cores while tile t-1 is converted and stored.
    f32x16 ka[2], va[2];
    // The h fragments of tile t + 1 are requested before the products of tile t,
    // so the LDS latency hides behind 2 KD matrix instructions.
    f16x8 hf[2][KD];
    auto fetch = [&](int t, int buf) {
#pragma unroll
      for (int kk = 0; kk < KD; ++kk)
        hf[buf][kk] = BLK ? tile_chunk<D>(rX + t * P::TILEB, li, 2 * kk + g) : Hb[(t * KD + kk) * 64 + lane];
    };
    // Token tiles in the order w, w + 1, .. (mod 4): step i projects tile tile_of(i).
    auto tile_of = [&](int i) { return (i + w) & (kSplitTiles - 1); };
    // Step i - 1's tile is converted and stored a quarter at a time between the products
    // of step i, each quarter pinned after two products (scheduling barriers): the wave
    // issues instructions in order, so conversions placed after a run of products
    // would leave the matrix cores idle while they execute.
    auto store_part = [&](int i, int c) {  // c: K half 0, K half 1, V half 0, V half 1
      const int half = c & 1, t = tile_of(i);
      const f16x8 o = acc_f16(c < 2 ? ka[i & 1] : va[i & 1], half);
      if constexpr (P::NARROW) {
        if (c < 2)
          Kl[(t * KD + 2 * w + half) * 64 + lane] = o;
        else
          Vl[((t * NNT + w) * 2 + half) * 64 + lane] = o;
      } else {
        if (c < 2)
          Kl[((h * kSplitTiles + t) * KSH + 2 * t2 + half) * 64 + lane] = o;
        else
          Vl[(((h * kSplitTiles + t) * NDT + t2) * 2 + half) * 64 + lane] = o;
      }
    };
    auto products = [&](int i) {
      if (doq && i + 1 < kSplitTiles) issue_wq(i);
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) {
        const f16x8 hb = hf[i & 1][kk];
        ka[i & 1] = mfma32x32x16(wk[kk], hb, kk == 0 ? bk : ka[i & 1]);
        va[i & 1] = mfma32x32x16(hb, wv[kk], kk == 0 ? bv : va[i & 1]);
        // The next tile's fragments (after the last tile: those of the slice, for
        // Q^T) are requested behind this tile's first two products, never ahead of
        // them.  The first wait for LDS data after an LDS-DMA issue (issue_wq) is
        // compiled as lgkmcnt(0), i.e. it would also wait for requests just made.
        // Step 0 runs before the barrier: the next tile is another wave's.
        if (kk == 0 && i > 0) {
          __builtin_amdgcn_sched_barrier(0);
          fetch(i + 1 < kSplitTiles ? tile_of(i + 1) : s, (i + 1) & 1);
          // The W_q rows (this wave's own transfers, issued two tiles ago at the latest).
          if (doq && i + 1 == kSplitTiles) {
            wait_vmcnt<0>();
#pragma unroll
            for (int dt = 0; dt < NQT; ++dt)
#pragma unroll
              for (int k2 = 0; k2 < KD; ++k2) wq[dt][k2] = tile_chunk<D>(rWq, 32 * dt + li, 2 * k2 + g);
          }
        }
        if (i >= 1)
#pragma unroll
          for (int c = kk * 4 / KD; c < (kk + 1) * 4 / KD; ++c) store_part(i - 1, c);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    fetch(tile_of(0), 0);
    products(0);
    lds_barrier();  // LN1 output of every tile is in LDS; every wave has its weight fragments
    fetch(tile_of(1), 1);
#pragma unroll
    for (int i = 1; i < kSplitTiles; ++i) products(i);
    // Q^T of the slice for head w (waves past the last head have none), or d-tile w
    // of the split head, with the last K / V tile stored between its products.
    if (doq) {
#pragma unroll
      for (int dt = 0; dt < NQT; ++dt) {
        f32x16 qa;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const f32x4 t = *reinterpret_cast<const f32x4*>(pp + 64 + 32 * dt + 8 * qd + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e) qa[4 * qd + e] = t[e];
        }
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
          qa = mfma32x32x16(wq[dt][kk], hf[kSplitTiles & 1][kk], qa);
          if (dt == 0)
#pragma unroll
            for (int c = kk * 4 / KD; c < (kk + 1) * 4 / KD; ++c) store_part(kSplitTiles - 1, c);
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          if constexpr (P::QSPLIT)
            Qx[(2 * w + half) * 64 + lane] = acc_f16(qa, half);  // k-steps 2w, 2w + 1 of the head
          else
            qB[2 * dt + half] = acc_f16(qa, half);
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) store_part(kSplitTiles - 1, c);
    }
  } else {
    lds_barrier();  // the products' barrier above: LN1 output of every tile is in LDS
  }
  // K, V of every token tile and head are in LDS; every W_q read is done.  At d_model 128
  // and head_dim 32 (outside the whole-block mode) no wave needs another's: wave w
  // projected exactly head w's K and V, runs head w's attention, and its W_q staging
  // area, which the W_o rows below overwrite, is its own.
  constexpr bool kOwnHead = D == 128 && HD == 32 && !BLK;
  if constexpr (!kOwnHead) lds_barrier();
  // W_o rows 32dq .. 32dq+31 into the W_q staging area, free now: they land during the
  // attention.  (Waves past the last output tile fetch tile 0 again, identical bytes
  // to the same place.)
  dma_span_rows<D, P::N_O>(rWo, reinterpret_cast<const char*>(wo + (int64_t)32 * dq * D), spans);

  // ---- attention of head w: S^T = K Q^T for all (at most 128) keys at once, one exact
  // softmax pass (no running max, no rescale), O^T = V^T P^T.
  if constexpr (P::QSPLIT) {
    // One head of 128 dims over four waves: wave w scores key tile w for the slice's
    // queries, the per-query max and sum of the four tiles meet in LDS, the
    // probabilities go to LDS as B-operand fragments, and wave w forms output d-tile w
    // over all keys.  (Stat is free until the LayerNorm below.)
    const int t = w;
    f16x8 kf[KSH], qf[KSH];
#pragma unroll
    for (int ks = 0; ks < KSH; ++ks) {
      kf[ks] = Kl[(t * KSH + ks) * 64 + lane];
      qf[ks] = Qx[ks * 64 + lane];
    }
    __builtin_amdgcn_sched_barrier(0);
    f32x16 sacc = zero16();
#pragma unroll
    for (int ks = 0; ks < KSH; ++ks) sacc = mfma32x32x16(kf[ks], qf[ks], sacc);
    if (32 * t + 32 > S || (CAUSAL && t >= s)) {
      int lim = S - 32 * t - 4 * g;  // valid: row offset < lim
      if (CAUSAL) lim = min(lim, qtok - 32 * t - 4 * g + 1);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) >= lim) sacc[r] = kNegInf;
    }
    if constexpr (MASKED) {
      if (kbits.tile(t) != 0xffffffffu) mask_key_tile(sacc, kbits.tile(t), g);
    }
    float mx = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
    mx = max_xor32(mx);
    if (g == 0) Stat[w * 32 + li] = mx;
    lds_barrier();  // every wave's tile max; every Q^T read is done
    mx = fmaxf(fmaxf(Stat[li], Stat[32 + li]), fmaxf(Stat[64 + li], Stat[96 + li]));
    // Unmasked, key 0 is valid for every query, so the max is finite; a query whose
    // keys are all padded gets max -inf, all-zero probabilities and a zero row.
    float m = mx * c2;
    if constexpr (MASKED) m = mx == kNegInf ? 0.f : m;
    f16x8 pB[2];
    float lp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 16; ++r) pB[r >> 3][r & 7] = (f16)__builtin_amdgcn_exp2f(fmaf(sacc[r], c2, -m));
    add_probs(pB[0], lp[0], lp[1]);  // the fp16 probabilities the P.V product consumes
    add_probs(pB[1], lp[2], lp[3]);
    const float lt = sum_xor32((lp[0] + lp[1]) + (lp[2] + lp[3]));
    if (g == 0) Stat[(kSplitWaves + w) * 32 + li] = lt;
#pragma unroll
    for (int half = 0; half < 2; ++half) Px[(2 * t + half) * 64 + lane] = pB[half];
    lds_barrier();  // probabilities and partial sums of every key tile
    f32x16 ot = zero16();
#pragma unroll
    for (int tt = 0; tt < kSplitTiles; ++tt)
#pragma unroll
      for (int half = 0; half < 2; ++half)
        ot = mfma32x32x16(Vl[((tt * NDT + w) * 2 + half) * 64 + lane], Px[(2 * tt + half) * 64 + lane], ot);
    const float* const ls = Stat + kSplitWaves * 32;
    const float l = (ls[li] + ls[32 + li]) + (ls[64 + li] + ls[96 + li]);
    const float inv = MASKED ? (l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f) : __builtin_amdgcn_rcpf(l);
#pragma unroll
    for (int half = 0; half < 2; ++half) Cx[(2 * w + half) * 64 + lane] = scaled_f16(ot, half, inv);
  } else if constexpr (P::NARROW) {
    // Four 8-dim heads per wave: head 4w + j lives in k-step 2w + j/2, elements 0-3
    // (j even) or 4-7 (j odd) of each lane's fragment (dims 4g .. 4g+3 and 8 + 4g ..
    // 8 + 4g + 3 of the k-step).  Zeroing the other head's elements of the K
    // fragment leaves this head's scores; the output rows of head j of the d-tile
    // are accumulator registers 4j .. 4j+3, taken from that head's O^T.
    f32x16 ofin;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      __builtin_amdgcn_sched_barrier(0);  // one head at a time (register pressure)
      const int ks = 2 * w + (j >> 1);
      f32x16 sacc[kSplitTiles];
      float mx = kNegInf;
#pragma unroll
      for (int t = 0; t < kSplitTiles; ++t) {
        f16x8 kf = Kl[(t * KD + ks) * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) kf[(j & 1) ? e : 4 + e] = (f16)0.0f;
        sacc[t] = mfma32x32x16(kf, qB[j >> 1], zero16());
        if (32 * t + 32 > S || (CAUSAL && t >= s)) {
          int lim = S - 32 * t - 4 * g;  // valid: row offset < lim
          if (CAUSAL) lim = min(lim, qtok - 32 * t - 4 * g + 1);
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (8 * (r >> 2) + (r & 3) >= lim) sacc[t][r] = kNegInf;
        }
        if constexpr (MASKED) {
          if (kbits.tile(t) != 0xffffffffu) mask_key_tile(sacc[t], kbits.tile(t), g);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[t][r]);
      }
      mx = max_xor32(mx);
      float m = mx * c2;
      if constexpr (MASKED) m = mx == kNegInf ? 0.f : m;
      f32x16 ot = zero16();
      float lp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < kSplitTiles; ++t) {
        f16x8 pB[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) pB[r >> 3][r & 7] = (f16)__builtin_amdgcn_exp2f(fmaf(sacc[t][r], c2, -m));
        add_probs(pB[0], lp[0], lp[1]);  // the fp16 probabilities the P.V product consumes
        add_probs(pB[1], lp[2], lp[3]);
#pragma unroll
        for (int half = 0; half < 2; ++half)
          ot = mfma32x32x16(Vl[((t * NNT + w) * 2 + half) * 64 + lane], pB[half], ot);
      }
      const float l = sum_xor32((lp[0] + lp[1]) + (lp[2] + lp[3]));
      const float inv = MASKED ? (l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f) : __builtin_amdgcn_rcpf(l);
#pragma unroll
      for (int e = 0; e < 4; ++e) ofin[4 * j + e] = ot[4 * j + e] * inv;
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) Cx[(2 * w + half) * 64 + lane] = acc_f16(ofin, half);
  } else if (w < H) {
    const int h = w;
    // Every K and V fragment of the head is requested up front; the scheduling
    // barrier keeps the requests ahead of the products that wait on them.
    f16x8 kf[kSplitTiles][KSH], vf[kSplitTiles][2][NDT];
#pragma unroll
    for (int t = 0; t < kSplitTiles; ++t)
#pragma unroll
      for (int ks = 0; ks < KSH; ++ks) kf[t][ks] = Kl[((h * kSplitTiles + t) * KSH + ks) * 64 + lane];
#pragma unroll
    for (int t = 0; t < kSplitTiles; ++t)
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) vf[t][half][dt] = Vl[(((h * kSplitTiles + t) * NDT + dt) * 2 + half) * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);
    f32x16 sacc[kSplitTiles];
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < kSplitTiles; ++t) {
      sacc[t] = zero16();
#pragma unroll
      for (int ks = 0; ks < KSH; ++ks) sacc[t] = mfma32x32x16(kf[t][ks], qB[ks], sacc[t]);
      // Keys past S and, causally, keys after the query.
      if (32 * t + 32 > S || (CAUSAL && t >= s)) {
        int lim = S - 32 * t - 4 * g;  // valid: row offset < lim
        if (CAUSAL) lim = min(lim, qtok - 32 * t - 4 * g + 1);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (8 * (r >> 2) + (r & 3) >= lim) sacc[t][r] = kNegInf;
      }
      if constexpr (MASKED) {
        if (kbits.tile(t) != 0xffffffffu) mask_key_tile(sacc[t], kbits.tile(t), g);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[t][r]);
    }
    mx = max_xor32(mx);
    // Unmasked, key 0 is valid for every query, so the max is finite; a query whose
    // keys are all padded gets max -inf, all-zero probabilities and a zero row.
    float m = mx * c2;
    if constexpr (MASKED) m = mx == kNegInf ? 0.f : m;
    f32x16 ot[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) ot[dt] = zero16();
    float lp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kSplitTiles; ++t) {
      f16x8 pB[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) pB[r >> 3][r & 7] = (f16)__builtin_amdgcn_exp2f(fmaf(sacc[t][r], c2, -m));
      // The row sum adds the fp16 probabilities the P.V product consumes (pair dot
      // products against ones, fp32 accumulation: half the vector instructions).
      add_probs(pB[0], lp[0], lp[1]);
      add_probs(pB[1], lp[2], lp[3]);
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) ot[dt] = mfma32x32x16(vf[t][half][dt], pB[half], ot[dt]);
    }
    const float l = sum_xor32((lp[0] + lp[1]) + (lp[2] + lp[3]));
    const float inv = MASKED ? (l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f) : __builtin_amdgcn_rcpf(l);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int half = 0; half < 2; ++half) Cx[(h * KSH + 2 * dt + half) * 64 + lane] = scaled_f16(ot[dt], half, inv);
  }
  wait_vmcnt<0>();  // W_o rows (this wave's own transfers: readable without a barrier)
  // Row li of the W_o tile at the k order of the attention output: columns
  // 16ks + 4g + {0..3} (chunk 2ks) and 16ks + 8 + 4g + {0..3} (chunk 2ks + 1).
  f16x8 wof[KD];
#pragma unroll
  for (int ks = 0; ks < KD; ++ks) {
    const char* row = rWo + li * 2 * D + 8 * g;
    const f16x4 lo = *reinterpret_cast<const f16x4*>(row + 16 * ((2 * ks) ^ row_swz<D>(li)));
    const f16x4 hi = *reinterpret_cast<const f16x4*>(row + 16 * ((2 * ks + 1) ^ row_swz<D>(li)));
    wof[ks] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  lds_barrier();    // attention output of every head is in LDS
  // Whole-block mode: W1 rows 32w .. 32w+31 (FFN hidden tile w) into the token-tile area,
  // free now; it lands during the out-projection and LN2.  (Issued before the attention
  // instead, it slowed the attention's LDS reads by more than the transfer saved.)  W2
  // follows after the LN2 exchange, so the two do not queue in front of each other.
  char* const rW1 = rX + w * P::TILEB;
  char* const rW2 = rQ + w * P::TILEB;
  if constexpr (BLK) dma_span_rows<D, P::N_O>(rW1, reinterpret_cast<const char*>(tail.w1 + (int64_t)32 * w * D), spans);

  // ---- out^T tile w = W_o[32w..32w+31] ctx^T, + b_o + x, then LN2 ----------------------
  float v[4][4];  // query qtok, column 32w + 8qd + 4g + e
  float sum = 0.f, sq = 0.f, pil2 = 0.f;
  if (w < NNT) {
    // Every attention-output fragment is requested before the first product (one wait).
    f16x8 cf[KD];
#pragma unroll
    for (int ks = 0; ks < KD; ++ks) cf[ks] = Cx[ks * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);
    f32x16 oacc = zero16();
#pragma unroll
    for (int ks = 0; ks < KD; ++ks) oacc = mfma32x32x16(wof[ks], cf[ks], oacc);
    // A padded query's attention output is zero (masked_fill before the residual add).
    const bool qv = !MASKED || kbits.valid(qtok);
    // LN2's pilot: column 0 of the row's input residual (x, or in the whole-block mode the
    // fp32 residual entering the block, wave 0's rows), the same value in every wave.
    pil2 = BLK ? *reinterpret_cast<const float*>(smem + P::OFF_R + li * 128 + 16 * (li & 7))
               : (float)reinterpret_cast<const f16*>(Raw + li)[0];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const f32x4 bb = *reinterpret_cast<const f32x4*>(pp + 128 + 8 * qd + 4 * g);
      // x[qtok][32w + 8qd + 4g + e]: k-step 2w + qd/2, fragment half qd % 2, elements 4g + e.
      float xr[4];
      if constexpr (BLK) {
        const f32x4 rr = *reinterpret_cast<const f32x4*>(rRes + li * 128 + 16 * ((2 * qd + g) ^ (li & 7)));
#pragma unroll
        for (int e = 0; e < 4; ++e) xr[e] = rr[e];
      } else {
        const f16x4 xh = *reinterpret_cast<const f16x4*>(
            reinterpret_cast<const char*>(Raw + (2 * w + (qd >> 1)) * 64 + li + 32 * (qd & 1)) + 8 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) xr[e] = (float)xh[e];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[qd][e] = (qv ? oacc[4 * qd + e] + bb[e] : 0.f) + xr[e];
        const float d = v[qd][e] - pil2;
        sum += d;
        sq = fmaf(d, d, sq);
      }
    }
    // LN2 statistics in one exchange: each wave's row sums and sums of squares of
    // d = r - pilot over its 32 columns; variance E[d^2] - E[d]^2 (the shift keeps it
    // well conditioned when the row's mean is large against its spread).
    sum = sum_xor32(sum);
    sq = sum_xor32(sq);
    if (g == 0) {
      Stat[w * 32 + li] = sum;
      Stat[(kSplitWaves + w) * 32 + li] = sq;
    }
  }
  lds_barrier();
  // W2 rows 32w .. 32w+31 (output tile w) into the W_o area (read into registers above).
  if constexpr (BLK) dma_span_rows<D, P::N_O>(rW2, reinterpret_cast<const char*>(tail.w2 + (int64_t)32 * w * D), spans);
  if (w < NNT) {
    float tot = 0.f, tsq = 0.f;
#pragma unroll
    for (int n = 0; n < NNT; ++n) {
      tot += Stat[n * 32 + li];
      tsq += Stat[(kSplitWaves + n) * 32 + li];
    }
    const float md = tot * (1.0f / D);
    const float rstd = rsqrtf(fmaxf(tsq * (1.0f / D) - md * md, 0.f) + eps);
    const float mean = pil2 + md;
    if constexpr (BLK) {
      // h2 = LN2(r1) rounded to fp16, into the attention-output area (read by every
      // wave's out-projection before the barrier above) as the B operand of the FFN:
      // k-step 2w + half holds columns 32w + 16 half + 4g + {0..3} and + 8.
      float o[4][4];
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f32x4 gg = *reinterpret_cast<const f32x4*>(pp + 160 + 8 * qd + 4 * g);
        const f32x4 bb = *reinterpret_cast<const f32x4*>(pp + 192 + 8 * qd + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[qd][e] = (v[qd][e] - mean) * rstd * gg[e] + bb[e];
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        f16x8 hh;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hh[e] = (f16)o[2 * half][e];
          hh[4 + e] = (f16)o[2 * half + 1][e];
        }
        Cx[(2 * w + half) * 64 + lane] = hh;
      }
    } else {
      // y of columns 32w + 8qd + 4g + {0..3}.  The lanes of a pair (g = 0, 1) hold one
      // row; one v_permlane32_swap per dword regroups quads qd, qd + 1 so that lane g
      // owns the 8 contiguous columns 32w + 8 (qd + g) .. + 7 and writes them with one
      // 16-byte store (two stores per lane instead of four of 8 bytes).  Every lane of the
      // pair takes part in the swap, stored row or not.
      const int64_t row = (int64_t)b * S + qtok;
#pragma unroll
      for (int qp = 0; qp < 4; qp += 2) {
        f16x4 yh[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int qd = qp + j;
          const f32x4 gg = *reinterpret_cast<const f32x4*>(pp + 160 + 8 * qd + 4 * g);
          const f32x4 bb = *reinterpret_cast<const f32x4*>(pp + 192 + 8 * qd + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e) yh[j][e] = (f16)((v[qd][e] - mean) * rstd * gg[e] + bb[e]);
        }
        swap_halves(yh[0], yh[1]);
        if (q_ok) {
          const f16x8 y8 = {yh[0][0], yh[0][1], yh[0][2], yh[0][3], yh[1][0], yh[1][1], yh[1][2], yh[1][3]};
          *reinterpret_cast<f16x8*>(y + row * D + 32 * w + 8 * (qp + g)) = y8;
        }
      }
      if (q_ok && resid_out) {
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) store4(resid_out + row * D + 32 * w + 8 * qd + 4 * g, v[qd]);
      }
    }
  }
  if constexpr (!BLK) return;

  // ---- whole-block mode: FFN and the next norm (TTB:1255-1267) ----------------------------
  // Row li of a W1 / W2 tile at the k order of the fragments the accumulators produce
  // (the same order as the W_o rows above).
  auto row_frags = [&](const char* tile, f16x8 (&f)[KD]) {
#pragma unroll
    for (int ks = 0; ks < KD; ++ks) {
      const char* row = tile + li * 2 * D + 8 * g;
      const f16x4 lo = *reinterpret_cast<const f16x4*>(row + 16 * ((2 * ks) ^ row_swz<D>(li)));
      const f16x4 hi = *reinterpret_cast<const f16x4*>(row + 16 * ((2 * ks + 1) ^ row_swz<D>(li)));
      f[ks] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  };
  const float* pt = reinterpret_cast<const float*>(rP + 1024);  // b1 | b2 | gn | bn of tile w
  f16x8* const Hid = Kl;  // FFN hidden fragments, in the K / V area (free after the attention)
  // The bias rows of this lane's accumulator registers (4qd + e: row 8qd + 4g + e), in
  // registers before the products rather than one LDS round trip per element after them.
  f32x4 b1v[4], b2v[4];
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    b1v[qd] = *reinterpret_cast<const f32x4*>(pt + 8 * qd + 4 * g);
    b2v[qd] = *reinterpret_cast<const f32x4*>(pt + 32 + 8 * qd + 4 * g);
  }
  wait_vmcnt<P::N_O>();    // W1 rows (W2 may still be in flight)
  f16x8 w1f[KD];
  row_frags(rW1, w1f);
  lds_barrier();  // h2 of every column tile is in LDS
  {
    // hid^T tile w = W1[32w .. 32w+31] h2^T, + b1, exact GELU, fp16 (TTB:1260).  Every
    // operand fragment is requested before the first product, so one wait covers them.
    f16x8 hb[KD];
#pragma unroll
    for (int ks = 0; ks < KD; ++ks) hb[ks] = Cx[ks * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);
    f32x16 acc = zero16();
#pragma unroll
    for (int ks = 0; ks < KD; ++ks) acc = mfma32x32x16(w1f[ks], hb[ks], acc);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      f16x8 hh;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = 8 * half + j;
        hh[j] = (f16)gelu_erf_fast(acc[r] + b1v[r >> 2][r & 3]);
      }
      Hid[(2 * w + half) * 64 + lane] = hh;
    }
  }
  wait_vmcnt<0>();  // W2 rows
  f16x8 w2f[KD];
  row_frags(rW2, w2f);
  lds_barrier();  // hidden activations of every tile are in LDS
  // r2 = (r1 + hid W2^T + b2) * row_valid (TTB:144-145), then the next norm, its
  // statistics shifted by LN2's pilot (0 on a padded row, whose r2 is 0).
  const float rv = (!MASKED || kbits.valid(qtok)) ? 1.f : 0.f;
  const float pil3 = pil2 * rv;
  sum = 0.f;
  sq = 0.f;
  {
    f16x8 hf2[KD];
#pragma unroll
    for (int ks = 0; ks < KD; ++ks) hf2[ks] = Hid[ks * 64 + lane];
    __builtin_amdgcn_sched_barrier(0);
    f32x16 acc = zero16();
#pragma unroll
    for (int ks = 0; ks < KD; ++ks) acc = mfma32x32x16(w2f[ks], hf2[ks], acc);
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const f32x4 bb = b2v[qd];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[qd][e] = (acc[4 * qd + e] + bb[e] + v[qd][e]) * rv;
        const float d = v[qd][e] - pil3;
        sum += d;
        sq = fmaf(d, d, sq);
      }
    }
  }
  sum = sum_xor32(sum);
  sq = sum_xor32(sq);
  if (g == 0) {
    Stat[w * 32 + li] = sum;
    Stat[(kSplitWaves + w) * 32 + li] = sq;
  }
  lds_barrier();
  float tot = 0.f, tsq = 0.f;
#pragma unroll
  for (int n = 0; n < NNT; ++n) {
    tot += Stat[n * 32 + li];
    tsq += Stat[(kSplitWaves + n) * 32 + li];
  }
  const float md = tot * (1.0f / D);
  const float rstd = rsqrtf(fmaxf(tsq * (1.0f / D) - md * md, 0.f) + eps);
  const float mean = pil3 + md;
  const float om = tail.mask_out ? rv : 1.f;
  const int64_t row = (int64_t)b * S + qtok;
  float o[4][4];
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const f32x4 gg = *reinterpret_cast<const f32x4*>(pt + 64 + 8 * qd + 4 * g);
    const f32x4 bb = *reinterpret_cast<const f32x4*>(pt + 96 + 8 * qd + 4 * g);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[qd][e] = ((v[qd][e] - mean) * rstd * gg[e] + bb[e]) * om;
  }
  if (tail.y_f32) {
    if (q_ok) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) store4(static_cast<float*>(yv) + row * D + 32 * w + 8 * qd + 4 * g, o[qd]);
    }
  } else {
    // fp16 y 16 bytes per lane, regrouped across the lane pair as in the sublayer's
    // epilogue above (every lane takes part in the swap).
#pragma unroll
    for (int qp = 0; qp < 4; qp += 2) {
      f16x4 yh[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) yh[j][e] = (f16)o[qp + j][e];
      swap_halves(yh[0], yh[1]);
      if (q_ok) {
        const f16x8 y8 = {yh[0][0], yh[0][1], yh[0][2], yh[0][3], yh[1][0], yh[1][1], yh[1][2], yh[1][3]};
        *reinterpret_cast<f16x8*>(y + row * D + 32 * w + 8 * (qp + g)) = y8;
      }
    }
  }
  if (q_ok) {
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) store4(resid_out + row * D + 32 * w + 8 * qd + 4 * g, v[qd]);
  }
}

bool layer_split_ok(int64_t seq_len, int64_t d_model, int64_t heads) {
  if (heads <= 0 || d_model % heads != 0 || seq_len < 1 || seq_len > kSmallMaxS) return false;
  const int64_t hd = d_model / heads;
  return (d_model == 128 && (hd == 8 || hd == 32 || hd == 64 || hd == 128)) ||
         (d_model == 64 && (hd == 32 || hd == 64));
}

bool layer_split_pays(int64_t batch, int64_t seq_len, int64_t d_model, int x_dtype) {
  // fp16 activations at d_model 64 / 128, and at most two rounds of workgroups;
  // beyond that the persistent kernel, which projects K and V once per
  // sequence, does less work per output.
  if (x_dtype != kF16 || (d_model != 64 && d_model != 128)) return false;
  const int64_t items = batch * ((seq_len + 31) / 32);
  return items <= 2 * (int64_t)compute_units();
}

// The launch of one call, resolved once: kernel variant (with and without a token mask)
// and argument block; x, y, the mask and the residual output are filled in per launch.
template <int D, int HD, bool CAUSAL>
static void prepare_split(const SmallLayerArgs& a, float c2, SplitLaunch* l) {
  const bool aff1 = a.ln1_w != nullptr;
  l->fn[0] = aff1 ? (const void*)layer_split_kernel<D, HD, CAUSAL, false, false, true>
                  : (const void*)layer_split_kernel<D, HD, CAUSAL, false, false, false>;
  l->fn[1] = aff1 ? (const void*)layer_split_kernel<D, HD, CAUSAL, true, false, true>
                  : (const void*)layer_split_kernel<D, HD, CAUSAL, true, false, false>;
  l->grid = (unsigned)(a.batch * ((a.seq_len + 31) / 32));
  SplitArgs& k = l->args;
  k = SplitArgs{(int)a.seq_len, (int)l->grid, static_cast<const f16*>(a.x), static_cast<const f16*>(a.w_qkv),
                a.b_qkv, a.b_o, a.ln2_w, a.ln2_b, static_cast<const f16*>(a.w_o), a.ln1_w, a.ln1_b, a.y,
                a.resid_out, c2, a.eps, a.valid_mask};
}

template <bool CAUSAL>
static void split_shape(const SmallLayerArgs& a, float c2, SplitLaunch* l) {
  const int64_t hd = a.d_model / a.heads;
  if (a.d_model == 128) {
    if (hd == 8) return prepare_split<128, 8, CAUSAL>(a, c2, l);
    if (hd == 32) return prepare_split<128, 32, CAUSAL>(a, c2, l);
    if (hd == 64) return prepare_split<128, 64, CAUSAL>(a, c2, l);
    return prepare_split<128, 128, CAUSAL>(a, c2, l);
  }
  return hd == 32 ? prepare_split<64, 32, CAUSAL>(a, c2, l) : prepare_split<64, 64, CAUSAL>(a, c2, l);
}

bool layer_split_takes(const SmallLayerArgs& a) {
  return layer_split_ok(a.seq_len, a.d_model, a.heads) && layer_split_pays(a.batch, a.seq_len, a.d_model, a.x_dtype);
}

static float split_c2(const SmallLayerArgs& a) {
  const double hd = (double)(a.d_model / a.heads);
  return (float)(1.0 / sqrt(hd)) * 1.4426950408889634f;
}

bool prepare_layer_split(const SmallLayerArgs& a, SplitLaunch* l) {
  if (!layer_split_takes(a) || a.batch < 1 || a.batch * ((a.seq_len + 31) / 32) > 0x7fffffff) return false;
  const float c2 = split_c2(a);
  l->block = 64 * kSplitWaves;
  if (a.causal)
    split_shape<true>(a, c2, l);
  else
    split_shape<false>(a, c2, l);
  return true;
}

hipError_t launch_layer_split(const SplitLaunch& l, const void* x, const uint8_t* valid_mask, void* y,
                              float* resid_out, hipStream_t stream) {
  SplitArgs k = l.args;
  k.x = static_cast<const f16*>(x);
  k.vmask = valid_mask;
  k.y = y;
  k.resid_out = resid_out;
  void* args[] = {&k.S, &k.nblk, &k.x, &k.wqkv, &k.bqkv, &k.bo, &k.g2, &k.be2, &k};
  return hipLaunchKernel(l.fn[valid_mask ? 1 : 0], dim3(l.grid), dim3(l.block), args, 0, stream);
}

hipError_t run_layer_split(const SmallLayerArgs& a) {
  SplitLaunch l;
  if (!prepare_layer_split(a, &l)) return hipErrorInvalidValue;
  return launch_layer_split(l, a.x, a.valid_mask, a.y, a.resid_out, a.stream);
}

// ---- whole-block mode -------------------------------------------------------------------

bool block_split_ok(int64_t seq_len, int64_t d_model, int64_t heads, int64_t ffn_dim) {
  return d_model == 128 && ffn_dim == 128 && layer_split_ok(seq_len, d_model, heads);
}

bool block_split_pays(int64_t batch, int64_t seq_len) {
  return batch * ((seq_len + 31) / 32) <= 2 * (int64_t)compute_units();
}

template <int HD, bool CAUSAL>
static hipError_t launch_block(const BlockArgs& a, float c2) {
  const int64_t grid = a.batch * ((a.seq_len + 31) / 32);
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  SplitKArgs<true> k;
  static_cast<SplitArgs&>(k) =
      SplitArgs{(int)a.seq_len, (int)grid, static_cast<const f16*>(a.h), static_cast<const f16*>(a.w_qkv), a.b_qkv,
                a.b_o, a.ln2_w, a.ln2_b, static_cast<const f16*>(a.w_o), nullptr, nullptr, a.out, a.r_out, c2, a.eps,
                a.valid_mask};
  k.tail = BlockTail{a.r, static_cast<const f16*>(a.w1), a.b1, static_cast<const f16*>(a.w2), a.b2, a.lnn_w,
                     a.lnn_b, a.out_dtype == kF32, a.mask_out};
  auto kern = a.valid_mask ? layer_split_kernel<128, HD, CAUSAL, true, true, false>
                           : layer_split_kernel<128, HD, CAUSAL, false, true, false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * kSplitWaves), 0, a.stream, k.S, k.nblk, k.x, k.wqkv,
                     k.bqkv, k.bo, k.g2, k.be2, k);
  return hipGetLastError();
}

template <bool CAUSAL>
static hipError_t block_shape(const BlockArgs& a, float c2) {
  switch (a.d_model / a.heads) {
    case 8: return launch_block<8, CAUSAL>(a, c2);
    case 32: return launch_block<32, CAUSAL>(a, c2);
    case 64: return launch_block<64, CAUSAL>(a, c2);
    default: return launch_block<128, CAUSAL>(a, c2);
  }
}

hipError_t run_block_split(const BlockArgs& a) {
  if (!block_split_ok(a.seq_len, a.d_model, a.heads, a.ffn_dim) || a.batch < 0 || a.batch > 0x7fffffff)
    return hipErrorInvalidValue;
  if (a.batch == 0) return hipSuccess;
  const double hd = (double)(a.d_model / a.heads);
  const float c2 = (float)(1.0 / sqrt(hd)) * 1.4426950408889634f;  // as the sublayer mode
  return a.causal ? block_shape<true>(a, c2) : block_shape<false>(a, c2);
}

}  // namespace cobra
