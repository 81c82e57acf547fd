// The whole attention sublayer in one kernel, split by query slices so that a
// small batch still covers the chip: workgroup (b, s) produces the outputs of
// queries 32s .. 32s+31 of sequence b (S <= 128, d_model <= 128, head_dim in
// {32, 64}; the same shapes as the persistent fused kernel).
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
//   1. wave w loads, straight into registers, the W_k / W_v rows of d-tile w,
//      the W_q rows of head w and the W_o rows of output tile w, and
//      normalises tokens 32w .. 32w+31 (LN1) into LDS while those loads fly;
//   2. wave w projects K^T and V of d-tile w for ALL tokens (every workgroup
//      of the sequence recomputes them: twice the projection FLOPs of the
//      persistent kernel, but no cross-workgroup traffic at all), and Q^T of
//      the slice for head w;
//   3. wave h runs the attention of head h over all keys; the softmax is
//      exact, every key of the sequence is present;
//   4. wave n multiplies the gathered attention output by the W_o rows of
//      output columns 32n .. 32n+31, adds bias and residual, and LN2 combines
//      the per-wave row sums through LDS.
// Every global access is a plain load issued from straight-line code, so the
// compiler's wait counts stay exact and nothing waits on a transfer it does
// not need.
#include "common.hpp"
#include "kernels.hpp"
#include "layer_common.hpp"

namespace cobra {

namespace {

constexpr int kSplitWaves = 4;
constexpr int kSplitTiles = kSmallMaxS / 32;  // token tiles of a sequence

// LDS plan, in 1 KB chunk rows (64 lanes x 16 bytes, one operand fragment each).
template <int D, int HD>
struct SplitLds {
  static constexpr int KD = D / 16;    // k-steps over d_model
  static constexpr int NNT = D / 32;   // 32-wide tiles of d_model
  static constexpr int H = D / HD;
  static constexpr int NDT = HD / 32;  // 32-wide d tiles per head
  static constexpr int KSH = HD / 16;  // k-steps per head
  static constexpr int HB = kSplitTiles * KD;            // LN1 output (token tile, k-step)
  static constexpr int KT = H * kSplitTiles * KSH;       // K^T fragments (head, key tile, k-step)
  static constexpr int VT = H * kSplitTiles * NDT * 2;   // V fragments (head, key tile, d tile, half)
  static constexpr int CTX = KD;                         // attention output of the slice
  static constexpr int LN1P = kSplitWaves;               // per-wave copy of [gamma1 | beta1]
  static constexpr int ROWS = HB + KT + VT + CTX + LN1P;
  static constexpr int STAT = 2 * kSplitWaves * 32;      // LN2 partial sums (pass, wave, query), floats
  static_assert(D % 32 == 0 && HD % 32 == 0 && D % HD == 0, "layout");
  static_assert(H <= kSplitWaves && NNT <= kSplitWaves, "one wave per head and per d / output tile");
  static_assert(2 * D * 4 <= 1024, "LN1 parameters of one wave fit one 1 KB row");
  static_assert(ROWS * 1024 + STAT * 4 <= kLdsBytes, "LDS budget");
};

}  // namespace

template <int D, int HD, bool CAUSAL, typename TX>
__global__ __launch_bounds__(64 * kSplitWaves) void layer_split_kernel(
    const TX* __restrict__ x, const f16* __restrict__ wqkv, const float* __restrict__ bqkv,
    const f16* __restrict__ wo, const float* __restrict__ bo, const float* __restrict__ g1,
    const float* __restrict__ be1, const float* __restrict__ g2, const float* __restrict__ be2, TX* __restrict__ y,
    float* __restrict__ resid_out, int S, int NS, float c2, float eps) {
  using L = SplitLds<D, HD>;
  constexpr int KD = L::KD, NNT = L::NNT, H = L::H, NDT = L::NDT, KSH = L::KSH;
  using Raw8 = typename XChunks<TX>::c8;
  using Raw4 = typename XChunks<TX>::c4;

  __shared__ __attribute__((aligned(1024))) f16x8 lds[L::ROWS * 64 + L::STAT / 4];
  f16x8* const Hb = lds;                    // LN1 output of every token tile
  f16x8* const Kl = Hb + L::HB * 64;
  f16x8* const Vl = Kl + L::KT * 64;
  f16x8* const Cx = Vl + L::VT * 64;
  f16x8* const Pw = Cx + L::CTX * 64;       // LN1 parameters, one 1 KB row per wave
  float* const Stat = reinterpret_cast<float*>(Pw + L::LN1P * 64);

  const int b = blockIdx.x / NS;
  const int s = blockIdx.x - b * NS;  // query slice
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 31, g = lane >> 5;
  const int tok = 32 * w + li;   // token of this lane for LN1
  const int qtok = 32 * s + li;  // query of this lane for attention, out-projection, LN2
  const bool tok_ok = tok < S, q_ok = qtok < S;
  const TX* xs = x + (int64_t)b * S * D;

  // ---- 1. loads, in the order they are needed.  Waves past the last head or d-tile
  // load a valid row they do not use; rows past S load row 0 (S >= 1) and are
  // zeroed where used.
  // gamma1 | beta1: 16 bytes per lane, through this wave's own LDS row.
  f32x4 pv;
  {
    const int c = lane * 4;
    const float* src = c < D ? g1 + c : be1 + (c < 2 * D ? c - D : 0);
    pv = *reinterpret_cast<const f32x4*>(src);
  }
  // LN1 input: token tok, columns 16kk + 8g + e.
  Raw8 xin[KD];
  {
    const TX* xr = xs + (int64_t)(tok_ok ? tok : 0) * D + 8 * g;
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) xin[kk] = *reinterpret_cast<const Raw8*>(xr + 16 * kk);
  }
  // W_k / W_v rows of d-tile w: lane -> row 32w + li, columns 16kk + 8g .. +8 (the A
  // operand of K^T = W_k h^T and the B operand of V = h W_v^T).
  const int dq = w < NNT ? w : 0;
  f16x8 wk[KD], wv[KD];
  {
    const f16* wr = wqkv + (int64_t)(D + 32 * dq + li) * D + 8 * g;
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) {
      wk[kk] = *reinterpret_cast<const f16x8*>(wr + 16 * kk);
      wv[kk] = *reinterpret_cast<const f16x8*>(wr + (int64_t)D * D + 16 * kk);
    }
  }
  // W_q rows of head w (A operand of Q^T = W_q h^T): row 32(w*NDT + dt) + li.
  const int hq = w < H ? w : 0;
  f16x8 wq[NDT][KD];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int kk = 0; kk < KD; ++kk)
      wq[dt][kk] = *reinterpret_cast<const f16x8*>(wqkv + (int64_t)(32 * (hq * NDT + dt) + li) * D + 16 * kk + 8 * g);
  // W_o rows of output tile w (A operand of out^T = W_o ctx^T), in the k order of the
  // attention output: columns 16ks + 4g + {0..3, 8..11}; the halves are joined where used.
  f16x4 wlo[KD], whi[KD];
#pragma unroll
  for (int ks = 0; ks < KD; ++ks) {
    const f16* p = wo + (int64_t)(32 * dq + li) * D + 16 * ks + 4 * g;
    wlo[ks] = *reinterpret_cast<const f16x4*>(p);
    whi[ks] = *reinterpret_cast<const f16x4*>(p + 8);
  }
  // Residual: query qtok, columns 32w + 8qd + 4g + e (rows past S are never stored).
  Raw4 xres[4];
  {
    const TX* xr = xs + (int64_t)(q_ok ? qtok : 0) * D + 32 * dq + 4 * g;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) xres[qd] = *reinterpret_cast<const Raw4*>(xr + 8 * qd);
  }

  // ---- LN1 of token tok (columns 16kk + 8g + e) into the token tile's LDS rows --------
  Pw[w * 64 + lane] = __builtin_bit_cast(f16x8, pv);
  {
    float xv[KD][8];
    float sum = 0.f;
#pragma unroll
    for (int kk = 0; kk < KD; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xv[kk][e] = tok_ok ? (float)xin[kk][e] : 0.f;
        sum += xv[kk][e];
      }
    const float mean = (sum + __shfl_xor(sum, 32)) * (1.0f / D);
    float q = 0.f;
#pragma unroll
    for (int kk = 0; kk < KD; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = xv[kk][e] - mean;
        q += t * t;
      }
    const float rstd = rsqrtf((q + __shfl_xor(q, 32)) * (1.0f / D) + eps);
    const float* pw = reinterpret_cast<const float*>(Pw + w * 64);  // written by this wave
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) {
      float gv[8], bv[8];
      load8(pw + 16 * kk + 8 * g, gv);
      load8(pw + D + 16 * kk + 8 * g, bv);
      f16x8 h;
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = (f16)((xv[kk][e] - mean) * rstd * gv[e] + bv[e]);
      Hb[(w * KD + kk) * 64 + lane] = h;
    }
  }
  __syncthreads();  // LN1 output of every token tile is in LDS

  // ---- 2. K^T and V of d-tile w for every token tile; Q^T of the slice for head w ---
  if (w < NNT) {
    float bk[16], bv[16];
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(bqkv + D + 32 * w + 8 * qd + 4 * g);
#pragma unroll
      for (int e = 0; e < 4; ++e) bk[4 * qd + e] = t[e];
    }
    const float bvl = bqkv[2 * D + 32 * w + li];
#pragma unroll
    for (int r = 0; r < 16; ++r) bv[r] = bvl;
    const int h = (32 * w) / HD, t2 = w % NDT;  // head and d tile within the head
#pragma unroll
    for (int t = 0; t < kSplitTiles; ++t) {
      f32x16 ka = zero16(), va = zero16();
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) {
        const f16x8 hb = Hb[(t * KD + kk) * 64 + lane];
        ka = mfma32x32x16(wk[kk], hb, ka);
        va = mfma32x32x16(hb, wv[kk], va);
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        Kl[((h * kSplitTiles + t) * KSH + 2 * t2 + half) * 64 + lane] = half_to_f16(ka, half, bk);
        Vl[(((h * kSplitTiles + t) * NDT + t2) * 2 + half) * 64 + lane] = half_to_f16(va, half, bv);
      }
    }
  }
  f16x8 qB[KSH];
  if (w < H) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      f32x16 qa = zero16();
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) qa = mfma32x32x16(wq[dt][kk], Hb[(s * KD + kk) * 64 + lane], qa);
      float bq[16];
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f32x4 t = *reinterpret_cast<const f32x4*>(bqkv + 32 * (w * NDT + dt) + 8 * qd + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) bq[4 * qd + e] = t[e];
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) qB[2 * dt + half] = half_to_f16(qa, half, bq);
    }
  }
  __syncthreads();  // K, V of every token tile and head are in LDS

  // ---- 3b. attention of head w: S^T = K Q^T over two blocks of two key tiles, exact
  // softmax with one rescale between the blocks, O^T = V^T P^T.
  if (w < H) {
    const int h = w;
    f32x16 ot[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) ot[dt] = zero16();
    float m_run = 0.f, l = 0.f;
#pragma unroll
    for (int blk = 0; blk < kSplitTiles / 2; ++blk) {
      f32x16 sacc[2];
      float mx = kNegInf;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int t = 2 * blk + u;
        sacc[u] = zero16();
#pragma unroll
        for (int ks = 0; ks < KSH; ++ks)
          sacc[u] = mfma32x32x16(Kl[((h * kSplitTiles + t) * KSH + ks) * 64 + lane], qB[ks], sacc[u]);
        // Keys past S and, causally, keys after the query.
        if (32 * t + 32 > S || (CAUSAL && t >= s)) {
          int lim = S - 32 * t - 4 * g;  // valid: row offset < lim
          if (CAUSAL) lim = min(lim, qtok - 32 * t - 4 * g + 1);
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (8 * (r >> 2) + (r & 3) >= lim) sacc[u][r] = kNegInf;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[u][r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // Block 0 holds key 0, valid for every query, so its max is finite; a fully
      // masked later block leaves the running max as it is.
      const float m_new = blk == 0 ? mx * c2 : fmaxf(m_run, mx * c2);
      const float alpha = blk == 0 ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      f16x8 pB[2][2];
      float ps = 0.f;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[u][r], c2, -m_new));
          ps += pv;
          pB[u][r >> 3][r & 7] = (f16)pv;
        }
      if (blk == 0) {
        l = ps;
      } else {
        l = l * alpha + ps;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) ot[dt][r] *= alpha;
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
            ot[dt] = mfma32x32x16(Vl[(((h * kSplitTiles + 2 * blk + u) * NDT + dt) * 2 + half) * 64 + lane],
                                  pB[u][half], ot[dt]);
    }
    l += __shfl_xor(l, 32);
    const float inv = __builtin_amdgcn_rcpf(l);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int half = 0; half < 2; ++half) Cx[(h * KSH + 2 * dt + half) * 64 + lane] = scaled_f16(ot[dt], half, inv);
  }
  __syncthreads();  // attention output of every head is in LDS

  // ---- 4. out^T tile w = W_o[32w..32w+31] ctx^T, + b_o + x, then LN2 ------------------------
  float v[4][4];  // query qtok, column 32w + 8qd + 4g + e
  float sum = 0.f;
  if (w < NNT) {
    f32x16 oacc = zero16();
#pragma unroll
    for (int ks = 0; ks < KD; ++ks) {
      const f16x8 a = {wlo[ks][0], wlo[ks][1], wlo[ks][2], wlo[ks][3], whi[ks][0], whi[ks][1], whi[ks][2], whi[ks][3]};
      oacc = mfma32x32x16(a, Cx[ks * 64 + lane], oacc);
    }
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const f32x4 bb = *reinterpret_cast<const f32x4*>(bo + 32 * w + 8 * qd + 4 * g);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[qd][e] = oacc[4 * qd + e] + bb[e] + (float)xres[qd][e];
        sum += v[qd][e];
      }
    }
    sum += __shfl_xor(sum, 32);
    if (g == 0) Stat[w * 32 + li] = sum;
  }
  __syncthreads();
  float mean = 0.f;
#pragma unroll
  for (int n = 0; n < NNT; ++n) mean += Stat[n * 32 + li];
  mean *= 1.0f / D;
  if (w < NNT) {
    float q = 0.f;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float t = v[qd][e] - mean;
        q += t * t;
      }
    q += __shfl_xor(q, 32);
    if (g == 0) Stat[(kSplitWaves + w) * 32 + li] = q;
  }
  __syncthreads();
  if (w < NNT) {
    float var = 0.f;
#pragma unroll
    for (int n = 0; n < NNT; ++n) var += Stat[(kSplitWaves + n) * 32 + li];
    const float rstd = rsqrtf(var * (1.0f / D) + eps);
    if (q_ok) {
      const int64_t row = (int64_t)b * S + qtok;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int n0 = 32 * w + 8 * qd + 4 * g;
        const f32x4 gg = *reinterpret_cast<const f32x4*>(g2 + n0);
        const f32x4 bb = *reinterpret_cast<const f32x4*>(be2 + n0);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (v[qd][e] - mean) * rstd * gg[e] + bb[e];
        store4(y + row * D + n0, o);
        if (resid_out) store4(resid_out + row * D + n0, v[qd]);
      }
    }
  }
}

bool layer_split_pays(int64_t batch, int64_t seq_len) {
  // Up to two rounds of workgroups; beyond that the persistent kernel, which
  // projects K and V once per sequence, does less work per output.
  const int64_t items = batch * ((seq_len + 31) / 32);
  return items <= 2 * (int64_t)compute_units();
}

template <int D, int HD, bool CAUSAL, typename TX>
static hipError_t launch_split(const SmallLayerArgs& a, float c2) {
  const int ns = (int)((a.seq_len + 31) / 32);
  const int64_t grid = a.batch * ns;
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((layer_split_kernel<D, HD, CAUSAL, TX>), dim3((unsigned)grid), dim3(64 * kSplitWaves), 0,
                     a.stream, static_cast<const TX*>(a.x), static_cast<const f16*>(a.w_qkv), a.b_qkv,
                     static_cast<const f16*>(a.w_o), a.b_o, a.ln1_w, a.ln1_b, a.ln2_w, a.ln2_b,
                     static_cast<TX*>(a.y), a.resid_out, (int)a.seq_len, ns, c2, a.eps);
  return hipGetLastError();
}

template <int D, int HD, bool CAUSAL>
static hipError_t split_dtype(const SmallLayerArgs& a, float c2) {
  return a.x_dtype == kF16 ? launch_split<D, HD, CAUSAL, f16>(a, c2) : launch_split<D, HD, CAUSAL, float>(a, c2);
}

template <bool CAUSAL>
static hipError_t split_shape(const SmallLayerArgs& a, float c2) {
  const int64_t hd = a.d_model / a.heads;
  if (a.d_model == 128) {
    if (hd == 32) return split_dtype<128, 32, CAUSAL>(a, c2);
    return split_dtype<128, 64, CAUSAL>(a, c2);
  }
  if (a.d_model == 64) {
    if (hd == 32) return split_dtype<64, 32, CAUSAL>(a, c2);
    return split_dtype<64, 64, CAUSAL>(a, c2);
  }
  return split_dtype<96, 32, CAUSAL>(a, c2);
}

// Shape and dtype checks are the caller's (run_layer_small).
hipError_t run_layer_split(const SmallLayerArgs& a, float c2) {
  return a.causal ? split_shape<true>(a, c2) : split_shape<false>(a, c2);
}

}  // namespace cobra
