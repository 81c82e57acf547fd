// Fused QKV projection + exact attention for wide heads of short sequences: one
// workgroup per (sequence, head), head_dim 256, S <= 128.
//
//   q, k, v = h W_{q,k,v}[head]^T + b;   ctx[:, head] = softmax(q k^T * scale) v
//
// The counterpart of the reference's _qkvattn_kernel (torch_transformer_benchmark.py:
// 654-741), which the reference takes when one query block covers the sequence
// (TTB:1030-1071): the projection runs inside the attention kernel, so q / k / v never
// reach memory.  Against a QKV GEMM followed by an attention kernel this saves the
// qkv round trip (3 T D fp16 written and read back: 100 MB at B64 d1024) and the
// GEMM's second round of output tiles; the projection FLOPs are the same, each
// (sequence, head) projecting only its own 768 columns.
//
// Eight waves (two per SIMD), two phases:
//   A. one k-loop over d_model (32-wide k-tiles, two LDS-DMA stages holding the
//      sequence's h rows and the head's W_q / W_k / W_v rows) in which wave w owns 64
//      rows of [W_q; W_k]_head -- Q^T for w < 4, K^T for w >= 4 -- against all 128
//      token slots (eight 32x32 accumulators) and V of d-tile w (four more, h as the A
//      operand).  Q^T and K^T go to LDS as fp16 operand fragments, bias added; V's
//      accumulator layout is the A operand of O^T = V^T P^T in the probabilities' key
//      order, so V stays in registers as fp16.  (Projecting V in a second k-loop read
//      h twice and paid the per-k-tile barrier and fragment latency twice over.)
//   B. S^T = K Q^T: wave w scores query tile w % 4 against key tiles 2 (w / 4) and
//      2 (w / 4) + 1 over all 256 dims; the two halves of a query's keys meet in LDS
//      for the row max, the fp16 probabilities go to LDS as the B operand of the
//      P.V product and the partial row sums alongside (the softmax is exact: every
//      key is present, one pass, no rescale); wave w then forms output d-tile w for
//      all four query tiles and stores ctx.
// Operand conventions as in common.hpp.  Rows past S read row S - 1 (finite); their
// keys get probability 0 and their queries are never stored.  h, the weights and ctx
// are fp16 or bf16 (a template type: v_mfma_f32_32x32x16_bf16 and bf16 probabilities
// for the latter), everything else is the same code.
#include "common.hpp"
#include "kernels.hpp"
#include "layer_common.hpp"
#include "lds_dma.hpp"

namespace cobra {

namespace {

constexpr int kQaWaves = 8;                   // 512 threads, two waves per SIMD
constexpr int kQaHd = 256;                    // head_dim
constexpr int kQaTok = 128;                   // token slots of a sequence
constexpr int kQaBk = 32;                     // d_model columns per k-tile: two 16-deep k-steps
constexpr int kQaRowB = kQaBk * 2;            // bytes of one k-tile row
// Stage: token rows 0..127, then the head's W_q, W_k and W_v rows (768).
constexpr int kQaRows = kQaTok + 3 * kQaHd;
constexpr int kQaStage = kQaRows * kQaRowB;         // 56 KB
constexpr int kQaLpt = kQaStage / 1024 / kQaWaves;  // 1 KB transfers per wave per k-tile
constexpr int kQaStages = 2;
// LDS map (bytes).  The stages [0, 112 K); then K^T | Q^T fragments [0, 128 K) (4 token
// tiles x 16 k-steps x 1 KB each); then the probabilities [0, 32 K) (4 query tiles x 8
// key k-steps x 1 KB); the row max / sum exchange at [128 K, 130 K).
constexpr int kQaFrag = 4 * 16 * 1024;
constexpr int kQaOffK = 0, kQaOffQ = kQaFrag, kQaOffP = 0;
constexpr int kQaOffStat = 2 * kQaFrag;
constexpr int kQaLds = kQaOffStat + 2 * kQaWaves * 32 * 4;
static_assert(kQaStage % (1024 * kQaWaves) == 0, "whole transfers per wave");
static_assert(kQaStages * kQaStage <= kQaOffStat, "stages below the exchange area");
static_assert(kQaLds <= kLdsBytes, "LDS budget");
static_assert(kQaLpt < 64, "vmcnt range");

// Rows of a k-tile are 64 bytes (4 chunks of 16); chunk c of row R sits at chunk
// c ^ ((R >> 2) & 3), so the 16 rows one fragment read touches at one logical chunk
// hit 16 distinct 4-bank groups.
template <typename T>
__device__ __forceinline__ typename Op16<T>::V8 qa_frag(const char* stage, int row, int chunk) {
  return *reinterpret_cast<const typename Op16<T>::V8*>(stage + row * kQaRowB + 16 * (chunk ^ ((row >> 2) & 3)));
}

// Registers 8 half .. 8 half + 7 of an accumulator in the operand type.
template <typename T>
__device__ __forceinline__ typename Op16<T>::V8 acc_op(const f32x16& acc, int half) {
  typename Op16<T>::V8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (T)acc[8 * half + e];
  return o;
}

// a += p0 + p2 + p4 + p6, b += p1 + p3 + p5 + p7 in pairs (v_dot2 against ones), fp32 sums.
template <typename T>
__device__ __forceinline__ void add_probs_op(const typename Op16<T>::V8& p, float& a, float& b) {
  using V2 = typename Op16<T>::V2;
  const V2 one2 = {(T)1.0f, (T)1.0f};
  a = dot2(V2{p[0], p[1]}, one2, a);
  b = dot2(V2{p[2], p[3]}, one2, b);
  a = dot2(V2{p[4], p[5]}, one2, a);
  b = dot2(V2{p[6], p[7]}, one2, b);
}

}  // namespace

template <bool CAUSAL, bool MASKED, typename T>
__global__ __launch_bounds__(64 * kQaWaves) void qkv_attn_head_kernel(
    int S, int H, int D, int B, const T* __restrict__ h, const T* __restrict__ wqkv,
    const float* __restrict__ bqkv, T* __restrict__ ctx, float c2, const uint64_t* __restrict__ key_bits,
    int nwords, uint64_t* __restrict__ fill, int64_t nfill) {
  using V8 = typename Op16<T>::V8;
  using V4 = typename Op16<T>::V4;
  __shared__ __attribute__((aligned(1024))) char smem[kQaLds];
  // The statistics words the out-projection that follows expects unwritten.
  for (int64_t i = (int64_t)blockIdx.x * (64 * kQaWaves) + threadIdx.x; i < nfill; i += (int64_t)gridDim.x * 64 * kQaWaves)
    fill[i] = kRowLnUnset;

  // Consecutive ids share the head, so the workgroups on one XCD share that head's
  // 1.5 MB of weights in its L2.
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int hh = id / B;
  const int b = id - hh * B;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31, g = lane >> 5;
  const int KT = D / kQaBk;
  const T* hseq = h + (int64_t)b * S * D;
  const char* hbytes = reinterpret_cast<const char*>(hseq);
  const char* wbytes = reinterpret_cast<const char*>(wqkv);

  KeyBits kbits{~0ull, ~0ull};
  if constexpr (MASKED) {
    const uint64_t* kb = key_bits + (int64_t)b * nwords;
    kbits = {kb[0], nwords > 1 ? kb[1] : 0ull};
  }

  // DMA sources.  Transfer i of wave w fills band w + 8 i (rows 16 band .. +15 of the
  // stage); lane l fills row 16 band + l / 4, slot l % 4, i.e. logical chunk
  // (l % 4) ^ ((l >> 4) & 3).  Band 0 .. 7 (i = 0) are token rows, the rest weight rows.
  const int lrow = lane >> 2, lchunk = (lane & 3) ^ ((lane >> 4) & 3);
  const uint32_t tok_off = (uint32_t)((min(16 * w + lrow, S - 1) * D + 8 * lchunk) * 2);
  uint32_t woff[kQaLpt];
#pragma unroll
  for (int i = 1; i < kQaLpt; ++i) {
    const int rw = 16 * (w + kQaWaves * i) + lrow - kQaTok;  // row of [W_q; W_k; W_v]_head
    const int grow = (rw / kQaHd) * D + hh * kQaHd + rw % kQaHd;
    woff[i] = (uint32_t)(((int64_t)grow * D + 8 * lchunk) * 2);
  }
  auto issue = [&](int stage, int k0) {
    char* dst = smem + stage * kQaStage + 1024 * w;
    dma16(hbytes + 2 * k0 + tok_off, dst);
#pragma unroll
    for (int i = 1; i < kQaLpt; ++i) dma16(wbytes + 2 * k0 + woff[i], dst + 1024 * kQaWaves * i);
  };

  // ---- A: Q^T (waves 0-3) / K^T (waves 4-7) rows 64 (w % 4) .. + 63 of the head, and V
  // of d-tile w, for every token slot --------------------------------------------------------
  f32x16 acc[2][4], vacc[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    acc[0][tt] = zero16();
    acc[1][tt] = zero16();
    vacc[tt] = zero16();
  }
  issue(0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    wait_vmcnt<0>();  // this wave's part of tile kt
    stage_barrier();  // every wave's part has landed; tile kt - 1's stage is free
    if (kt + 1 < KT) issue((kt + 1) % kQaStages, (kt + 1) * kQaBk);
    const char* st = smem + (kt % kQaStages) * kQaStage;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int c = 2 * kk + g;
      V8 af[2], hf[4], vf;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) af[dt] = qa_frag<T>(st, kQaTok + 64 * w + 32 * dt + li, c);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) hf[tt] = qa_frag<T>(st, 32 * tt + li, c);
      vf = qa_frag<T>(st, kQaTok + 2 * kQaHd + 32 * w + li, c);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        acc[0][tt] = mfma32x32x16(af[0], hf[tt], acc[0][tt]);
        acc[1][tt] = mfma32x32x16(af[1], hf[tt], acc[1][tt]);
        vacc[tt] = mfma32x32x16(hf[tt], vf, vacc[tt]);
      }
    }
  }
  lds_barrier();  // every wave is done with the stages
  {
    // + bias, fp16, into the K^T / Q^T fragment areas: k-step ks = 2 (2 (w % 4) + dt) + half
    // of the head's 16, token tile tt (the A operand of S^T = K Q^T for K, the B operand for Q).
    const bool isq = w < 4;
    V8* const dstf = reinterpret_cast<V8*>(smem + (isq ? kQaOffQ : kQaOffK));
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int grow0 = (isq ? 0 : D) + hh * kQaHd + 64 * (w & 3) + 32 * dt;
      f32x4 bq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        bq[q] = bqkv ? *reinterpret_cast<const f32x4*>(bqkv + grow0 + 8 * q + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        f32x16 v = acc[dt][tt];
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] += bq[r >> 2][r & 3];
#pragma unroll
        for (int half = 0; half < 2; ++half)
          dstf[(tt * 16 + 2 * (2 * (w & 3) + dt) + half) * 64 + lane] = acc_op<T>(v, half);
      }
    }
  }
  // V^T fragments (+ bias of column li), key k-step 2 tt + half: the A operand of O^T.
  V8 vA[8];
  {
    const float bvl = bqkv ? bqkv[2 * D + hh * kQaHd + 32 * w + li] : 0.f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x16 v = vacc[tt];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] += bvl;
#pragma unroll
      for (int half = 0; half < 2; ++half) vA[2 * tt + half] = acc_op<T>(v, half);
    }
  }
  lds_barrier();

  // ---- B: S^T for query tile qt, key tiles 2 kh, 2 kh + 1 ------------------------------
  const int qt = w & 3, kh = w >> 2;
  const int qtok = 32 * qt + li;
  float* const smax = reinterpret_cast<float*>(smem + kQaOffStat);
  float* const ssum = smax + kQaWaves * 32;
  f32x16 sacc[2];
  {
    const V8* Kf = reinterpret_cast<const V8*>(smem + kQaOffK);
    const V8* Qf = reinterpret_cast<const V8*>(smem + kQaOffQ);
    V8 qf[16];
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) qf[ks] = Qf[(qt * 16 + ks) * 64 + lane];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kt = 2 * kh + j;
      sacc[j] = zero16();
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) sacc[j] = mfma32x32x16(Kf[(kt * 16 + ks) * 64 + lane], qf[ks], sacc[j]);
    }
  }
  float mx = kNegInf;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int kt = 2 * kh + j;
    // Keys past S and, causally, keys after the query.
    if (32 * kt + 32 > S || (CAUSAL && kt >= qt)) {
      int lim = S - 32 * kt - 4 * g;  // valid: row offset < lim
      if (CAUSAL) lim = min(lim, qtok - 32 * kt - 4 * g + 1);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) >= lim) sacc[j][r] = kNegInf;
    }
    if constexpr (MASKED) {
      if (kbits.tile(kt) != 0xffffffffu) mask_key_tile(sacc[j], kbits.tile(kt), g);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[j][r]);
  }
  mx = max_xor32(mx);
  if (g == 0) smax[w * 32 + li] = mx;
  lds_barrier();  // every S^T product is done (the K^T / Q^T fragments are dead); maxima visible
  mx = fmaxf(mx, smax[(w ^ 4) * 32 + li]);
  // Unmasked, key 0 is valid for every query (finite max); a query whose keys are all
  // padded gets max -inf, all-zero probabilities and a zero row.
  float m = mx * c2;
  if constexpr (MASKED) m = mx == kNegInf ? 0.f : m;
  {
    V8* const Pf = reinterpret_cast<V8*>(smem + kQaOffP);
    float lp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kt = 2 * kh + j;
      V8 pB[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) pB[r >> 3][r & 7] = (T)__builtin_amdgcn_exp2f(fmaf(sacc[j][r], c2, -m));
      add_probs_op<T>(pB[0], lp[0], lp[1]);
      add_probs_op<T>(pB[1], lp[2], lp[3]);
#pragma unroll
      for (int half = 0; half < 2; ++half) Pf[(qt * 8 + 2 * kt + half) * 64 + lane] = pB[half];
    }
    const float l = sum_xor32((lp[0] + lp[1]) + (lp[2] + lp[3]));
    if (g == 0) ssum[w * 32 + li] = l;
  }

  lds_barrier();  // the probabilities and row sums of every wave

  // ---- O^T (d-tile w) for every query tile, / row sum, -> ctx ----------------------------
  const V8* Pf = reinterpret_cast<const V8*>(smem + kQaOffP);
  T* const crow0 = ctx + (int64_t)b * S * D + hh * kQaHd + 32 * w;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    f32x16 o = zero16();
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) o = mfma32x32x16(vA[ks], Pf[(q4 * 8 + ks) * 64 + lane], o);
    const float l = ssum[q4 * 32 + li] + ssum[(q4 + 4) * 32 + li];
    const float inv = MASKED ? (l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f) : __builtin_amdgcn_rcpf(l);
    const int query = 32 * q4 + li;
    // Lane (li, g) holds columns 8q + 4g + {0..3} of its row; one v_permlane32_swap per
    // dword regroups quads q, q + 1 across the lane pair so that lane g writes the 8
    // contiguous columns 8 (q + g) .. + 7 with one 16-byte store (every lane swaps).
#pragma unroll
    for (int qp = 0; qp < 4; qp += 2) {
      V4 hv[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) hv[j][e] = (T)(o[4 * (qp + j) + e] * inv);
      swap_halves(hv[0], hv[1]);
      if (query < S) {
        const V8 h8 = {hv[0][0], hv[0][1], hv[0][2], hv[0][3], hv[1][0], hv[1][1], hv[1][2], hv[1][3]};
        *reinterpret_cast<V8*>(crow0 + (int64_t)query * D + 8 * (qp + g)) = h8;
      }
    }
  }
}

bool qkv_attn_head_ok(int64_t seq_len, int64_t heads, int64_t head_dim) {
  const int64_t D = heads * head_dim;
  // d_model in whole k-tiles; every weight-row offset (3 D rows of D fp16) fits 32 bits.
  return head_dim == kQaHd && seq_len >= 1 && seq_len <= kQaTok && heads >= 1 && D <= 16384;
}

template <bool CAUSAL, bool MASKED, typename T>
static hipError_t launch_qkv_attn_head(const QkvAttnArgs& a, float c2) {
  const int64_t grid = a.batch * a.heads;
  if (grid > 0x7fffffff || a.batch > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((qkv_attn_head_kernel<CAUSAL, MASKED, T>), dim3((unsigned)grid), dim3(64 * kQaWaves), 0,
                     a.stream, (int)a.seq_len, (int)a.heads, (int)(a.heads * a.head_dim), (int)a.batch,
                     static_cast<const T*>(a.h), static_cast<const T*>(a.w_qkv), a.b_qkv, static_cast<T*>(a.ctx), c2,
                     a.key_bits, (int)mask_words(a.seq_len), a.fill, a.fill ? a.nfill : (int64_t)0);
  return hipGetLastError();
}

template <typename T>
static hipError_t dispatch_qkv_attn_head(const QkvAttnArgs& a, float c2) {
  if (a.key_bits)
    return a.causal ? launch_qkv_attn_head<true, true, T>(a, c2) : launch_qkv_attn_head<false, true, T>(a, c2);
  return a.causal ? launch_qkv_attn_head<true, false, T>(a, c2) : launch_qkv_attn_head<false, false, T>(a, c2);
}

hipError_t run_qkv_attn_head(const QkvAttnArgs& a) {
  if (!qkv_attn_head_ok(a.seq_len, a.heads, a.head_dim) || a.batch < 0 || !(a.scale > 0.f) || a.nfill < 0)
    return hipErrorInvalidValue;
  if (a.dtype != kF16 && a.dtype != kBF16) return hipErrorInvalidValue;
  if (a.batch == 0) return hipSuccess;
  const float c2 = a.scale * 1.4426950408889634f;
  return a.dtype == kBF16 ? dispatch_qkv_attn_head<bf16>(a, c2) : dispatch_qkv_attn_head<f16>(a, c2);
}

}  // namespace cobra
