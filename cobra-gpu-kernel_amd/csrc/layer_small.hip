// The whole attention sublayer in ONE kernel for short sequences and narrow
// models (S <= 128, d_model <= 128, head_dim in {32, 64}): one wave per 32
// tokens, persistent workgroups that loop over sequences.
//
//   h = LN1(x);  q,k,v = h W^T + b;  ctx = softmax(q k^T * scale) v;
//   r = x + ctx W_o^T + b_o;  y = LN2(r)
//
// This is the fusion of the reference's _add_ln_kernel, _qkvattn_kernel and
// _gemm_ln_kernel (torch_transformer_benchmark.py:491-535, 654-741, 394-463),
// which the reference ran as three launches inside a CUDA graph; here nothing
// but x, the weights and y touches HBM.
//
// Every intermediate stays in the register layout the next matrix product
// consumes (v_mfma_f32_32x32x16_f16, conventions in common.hpp):
//   * LN1 is computed in the lane that owns token (lane % 32) and k-slice
//     8*(lane / 32) of each 16-wide k-step -- exactly the B operand of
//     Q^T = W_q h^T and K^T = W_k h^T, and the A operand of V = h W_v^T;
//   * the C layout of Q^T / K^T puts d-values {4g..4g+3, 8+4g..8+4g+3} of one
//     token in lane (token, g); that is the (k-permuted) operand layout of
//     S^T = K Q^T, so Q never leaves the registers and K is written to LDS as
//     ready-made 16-byte operand chunks for the other waves;
//   * the C layout of V holds, for one d, keys {4g.., 8+4g..} -- the A operand
//     of O^T = V^T P^T in the same key order as the probabilities, which come
//     straight from the S^T accumulators;
//   * O^T holds, per lane, one query and d-values in that same permuted order:
//     the B operand of out^T = W_o ctx^T.  out^T then holds 64 of the 128
//     values of one output row per lane (the rest in lane ^ 32), so LN2 is an
//     in-lane sum plus one lane-pair exchange.
// With all keys of the sequence present (S <= 128) the softmax is exact in one
// pass: no running max, no rescaling.
//
// All weights (W_qkv and W_o, 128 KB at d_model 128) are staged into LDS once
// per workgroup, already cut into the 16-byte per-lane operand chunks of the
// products above, so every matrix operand is one conflict-free ds_read_b128
// and no product waits on a global load.  Each workgroup then walks sequences
// blockIdx.x, blockIdx.x + gridDim.x, ... so the weights are loaded once per
// CU rather than once per sequence.
#include "common.hpp"
#include "kernels.hpp"
#include "layer_common.hpp"
#include "lds_dma.hpp"

namespace cobra {

// LDS plan of the fused kernel, in 16-byte chunks.  G sequence groups (four
// waves each) share the staged weights and have a K/V area each.
template <int D, int HD, int G = 1>
struct SmallLds {
  static constexpr int KD = D / 16;
  static constexpr int NDT = HD / 32;
  static constexpr int KSH = HD / 16;
  static constexpr int MAXT = kSmallMaxS / 32;
  static constexpr int WQKV = 3 * (D / 32) * KD * 64;
  static constexpr int WO = (D / 32) * KD * 64;
  static constexpr int KCH = MAXT * KSH * 64;
  static constexpr int VCH = MAXT * NDT * 2 * 64;
  static constexpr int CORE = WQKV + WO + G * (KCH + VCH);
  // Biases and LayerNorm parameters [b_qkv 3D | b_o | g1 | b1 | g2 | b2] = 8D
  // floats, kept in LDS too when they fit (otherwise read from global memory).
  static constexpr int PCH = 8 * D * 4 / 16;
  static constexpr bool PARAMS = (CORE + PCH) * 16 <= kLdsBytes;
  static constexpr int TOTAL = CORE + (PARAMS ? PCH : 0);
  static_assert(D % 32 == 0 && HD % 32 == 0 && D % HD == 0, "layout");
  static_assert(CORE * 16 <= kLdsBytes, "weights + K/V must fit the workgroup's LDS");
};

// Two sequences per workgroup (eight waves, two per SIMD) when the weights and
// two K/V areas fit the LDS: while one sequence's waves wait on a dependent
// product or a load, the other's issue -- a lone wave per SIMD leaves the matrix
// cores idle through every softmax and the vector ALUs idle through every product.
template <int D, int HD, typename TX>
constexpr int small_groups() {
  using L1 = SmallLds<D, HD, 1>;
  constexpr bool fits = (L1::WQKV + L1::WO + 2 * (L1::KCH + L1::VCH)) * 16 <= kLdsBytes;
  // fp32 activations need more registers than two waves per SIMD leave (they spill).
  // Wider models need more registers than two waves per SIMD leave (d_model 96
  // spills; at 128 the second K/V area also pushes the parameters out of the LDS,
  // and the pair measured slower than one sequence at a time).
  return sizeof(TX) == 2 && fits && D <= 64 ? 2 : 1;
}

// FULL: every lane's token is in range -- S equals the 32 * kSmallWaves token slots of a
// sequence's waves (a shorter S leaves the last wave's lanes past it, whose rows belong
// to the next sequence) -- one sequence per workgroup and no residual output, so the
// stores of a sequence are unconditional.  The compiler can
// then count them: at the next sequence's LN1 it waits for the prefetched input and for
// the stores whose data registers LN1 reuses, where behind a per-lane condition it
// waited for every store (~1 us per sequence at B10000).
template <int D, int HD, bool CAUSAL, bool MASKED, typename TX, int G, bool FULL>
__global__ __launch_bounds__(64 * kSmallWaves * G) void layer_small_kernel(const TX* __restrict__ x, const f16* __restrict__ wqkv,
                                                          const float* __restrict__ bqkv, const f16* __restrict__ wo,
                                                          const float* __restrict__ bo, const float* __restrict__ g1,
                                                          const float* __restrict__ be1, const float* __restrict__ g2,
                                                          const float* __restrict__ be2, TX* __restrict__ y,
                                                          float* __restrict__ resid_out, int B, int S, float c2,
                                                          float eps, const uint8_t* __restrict__ vmask) {
  using L = SmallLds<D, HD, G>;
  constexpr int KD = L::KD;     // k-steps over d_model
  constexpr int NH = D / HD;    // heads
  constexpr int NDT = L::NDT;   // 32-row d-tiles per head
  constexpr int KSH = L::KSH;   // k-steps per head in Q K^T
  constexpr int NNT = D / 32;   // 32-column output tiles
  constexpr int MAXT = L::MAXT;

  // [W_qkv chunks | W_o chunks | per group: K^T of head j | V of head j], all operand-ready.
  __shared__ f16x8 lds[L::TOTAL];
  f16x8* const Wl = lds;
  f16x8* const Wol = Wl + L::WQKV;

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave index, provably uniform
  const int w = wid % kSmallWaves, grp = wid / kSmallWaves;          // wave within its sequence group
  f16x8* const Kl = Wol + L::WO + grp * (L::KCH + L::VCH);
  f16x8* const Vl = Kl + L::KCH;
  const int li = lane & 31, g = lane >> 5;
  const int tok = w * 32 + li;
  static_assert(!FULL || G == 1, "FULL takes one sequence per workgroup");
  const bool tok_ok = FULL || tok < S;

  // ---- stage the weights: 64-chunk row r (one k-step of one 32-row tile) goes
  // to wave r % 4, so every trip count below is a compile-time constant:
  // W_qkv row (rt, kk): lane -> W[32rt + lane%32][16kk + 8(lane/32) .. +8]
  // W_o row (nt, ks):   lane -> W_o[32nt + lane%32][16ks + 4(lane/32) + {0..3, 8..11}]
  {
    constexpr int ROWS_Q = L::WQKV / 64, ROWS_O = L::WO / 64;
    constexpr int NW = kSmallWaves * G;
    constexpr int RQ = (ROWS_Q + NW - 1) / NW, RO = (ROWS_O + NW - 1) / NW;
    const f16* wq_lane = wqkv + (int64_t)(lane & 31) * D + 8 * (lane >> 5);
    const f16* wo_lane = wo + (int64_t)(lane & 31) * D + 4 * (lane >> 5);
    f16x8 tq[RQ], to[RO];
#pragma unroll
    for (int u = 0; u < RQ; ++u) {
      const int r = wid + NW * u;
      if (ROWS_Q % NW == 0 || r < ROWS_Q)
        tq[u] = *reinterpret_cast<const f16x8*>(wq_lane + (int64_t)(32 * (r / KD)) * D + 16 * (r % KD));
    }
#pragma unroll
    for (int u = 0; u < RO; ++u) {
      const int r = wid + NW * u;
      if (ROWS_O % NW == 0 || r < ROWS_O) {
        const f16* p = wo_lane + (int64_t)(32 * (r / KD)) * D + 16 * (r % KD);
        const f16x4 lo = *reinterpret_cast<const f16x4*>(p);
        const f16x4 hi = *reinterpret_cast<const f16x4*>(p + 8);
        to[u] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
#pragma unroll
    for (int u = 0; u < RQ; ++u)
      if (ROWS_Q % NW == 0 || wid + NW * u < ROWS_Q) Wl[(wid + NW * u) * 64 + lane] = tq[u];
#pragma unroll
    for (int u = 0; u < RO; ++u)
      if (ROWS_O % NW == 0 || wid + NW * u < ROWS_O) Wol[(wid + NW * u) * 64 + lane] = to[u];
  }
  float* const Pf = reinterpret_cast<float*>(lds + L::CORE);
  const bool aff1 = g1 != nullptr;  // LN1 with elementwise affine
  if constexpr (L::PARAMS) {
    const float* src[6] = {bqkv, bo, g1, be1, g2, be2};
    const int len[6] = {3 * D, D, D, D, D, D};
    int off = 0;
#pragma unroll
    for (int v = 0; v < 6; ++v) {
      if (src[v])  // null gamma1 / beta1: no LN1 affine, nothing to stage
        for (int i = 4 * (int)threadIdx.x; i < len[v]; i += 4 * 64 * kSmallWaves * G)
          *reinterpret_cast<f32x4*>(Pf + off + i) = *reinterpret_cast<const f32x4*>(src[v] + i);
      off += len[v];
    }
  }
  __syncthreads();

  using Raw8 = typename XChunks<TX>::c8;
  using Raw4 = typename XChunks<TX>::c4;
  // LN1 input (and token mask bytes) of the next sequence, loaded one sequence ahead.
  Raw8 xpre[KD];
  KeyBytes kpre{1, 1};
  auto load_ln1_input = [&](int sq) {
    if constexpr (FULL) {
      // Unconditional (see FULL): past the batch, sequence B - 1 is read again and unused.
      const int sqc = sq < B ? sq : B - 1;
      if constexpr (MASKED) kpre = load_key_bytes(vmask + (int64_t)sqc * S, S, lane);
      const TX* xr = x + ((int64_t)sqc * S + tok) * D + 8 * g;
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) xpre[kk] = *reinterpret_cast<const Raw8*>(xr + 16 * kk);
      return;
    }
    if constexpr (MASKED) {
      if (sq < B) kpre = load_key_bytes(vmask + (int64_t)sq * S, S, lane);
    }
    const TX* xr = x + ((int64_t)sq * S + tok) * D + 8 * g;
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) {
      if (tok_ok && sq < B) {
        xpre[kk] = *reinterpret_cast<const Raw8*>(xr + 16 * kk);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xpre[kk][e] = (TX)0.0f;
      }
    }
  };
  // Workgroup blk takes sequence groups blk, blk + gridDim.x, ...; group grp of it
  // handles sequence G * that + grp.  Every wave runs every trip (the barriers are
  // workgroup-wide): a group past the batch computes on zeros and stores nothing.
  const int ngroups = (B + G - 1) / G;
  load_ln1_input((int)blockIdx.x * G + grp);
  // FULL: the first sequence's input is waited for here, and each later one right after
  // the previous sequence's 2 NNT stores (below), so that on both edges into the loop it
  // is known complete and no wait for outstanding stores lands at the loop's head.  The
  // empty asm statements read the loaded registers: the compiler then counts the loads
  // as complete at these two points (an explicit s_waitcnt alone does not stop it from
  // scheduling the loads below the wait, after which the loop head waited as if they
  // were in flight -- on every later iteration, that drained the previous stores).
  auto input_complete = [&]() {
    struct Words {
      uint32_t u[sizeof(Raw8) / 4];
    };
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) {
      const Words wd = __builtin_bit_cast(Words, xpre[kk]);
#pragma unroll
      for (int i = 0; i < (int)(sizeof(Raw8) / 4); ++i) asm volatile("" ::"v"(wd.u[i]));
    }
    if constexpr (MASKED) asm volatile("" ::"v"((uint32_t)kpre.lo), "v"((uint32_t)kpre.hi));
  };
  if constexpr (FULL) {
    wait_vmcnt<0>();
    input_complete();
  }

  for (int sg = blockIdx.x; sg < ngroups; sg += gridDim.x) {
    const int seq = sg * G + grp;
    const bool live = G == 1 || seq < B;
    const int64_t row = (int64_t)seq * S + tok;
    KeyBits kbits{~0ull, ~0ull};
    if constexpr (MASKED) kbits = key_bits_of(kpre, S, lane);
    const float *gamma1, *beta1, *gamma2, *beta2, *bias_o, *bias_qkv;
    if constexpr (L::PARAMS) {
      bias_qkv = Pf;
      bias_o = Pf + 3 * D;
      gamma1 = Pf + 4 * D;
      beta1 = Pf + 5 * D;
      gamma2 = Pf + 6 * D;
      beta2 = Pf + 7 * D;
    } else {
      const int z = opaque_zero();
      bias_qkv = bqkv + z;
      bias_o = bo + z;
      gamma1 = g1 + z;
      beta1 = be1 + z;
      gamma2 = g2 + z;
      beta2 = be2 + z;
    }

    // ---- LN1: token `tok`, columns 16kk + 8g + e -------------------------------
    f16x8 hB[KD];
    if constexpr (sizeof(TX) == 2) {
      if (!aff1) {
        // fp16 input, no elementwise affine (the module's case): one pass over the row,
        // shifted by a pilot p (one element of the row, common to the lane pair): sums of
        // d = x - p and d^2 by fp16 pair dot products (exact products, fp32
        // accumulation), variance E[d^2] - E[d]^2, well conditioned also when the mean is
        // large against the spread; then h = x rstd - mean rstd as one mixed-precision fma
        // per element.  No fp32 copy of the row is formed, so LN1 needs few registers of
        // its own (with a 64-register copy, the compiler took the previous sequence's
        // store data registers and waited for those stores).
        const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
        const f16 pil = pair_pilot((f16)xpre[0][0]);
        const f16x2 p2 = {pil, pil};
        float s1[2] = {0.f, 0.f}, s2[2] = {0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KD; ++kk)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f16x2 pr = pk_sub_f16(f16x2{(f16)xpre[kk][2 * e], (f16)xpre[kk][2 * e + 1]}, p2);
            s1[e & 1] = __builtin_amdgcn_fdot2(pr, one2, s1[e & 1], false);
            s2[e & 1] = __builtin_amdgcn_fdot2(pr, pr, s2[e & 1], false);
          }
        const float md = sum_xor32(s1[0] + s1[1]) * (1.0f / D);
        const float ed2 = sum_xor32(s2[0] + s2[1]) * (1.0f / D);
        const float rstd = rsqrtf(fmaxf(ed2 - md * md, 0.f) + eps);
        const float mean = (float)pil + md;
        const float nmr = -mean * rstd;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk)
#pragma unroll
          for (int e = 0; e < 8; ++e) hB[kk][e] = (f16)fmaf((float)xpre[kk][e], rstd, nmr);
      }
    }
    if (sizeof(TX) != 2 || aff1) {
      float xv[KD][8];
      float s = 0.f;
#pragma unroll
      for (int kk = 0; kk < KD; ++kk) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xv[kk][e] = (float)xpre[kk][e];
          s += xv[kk][e];
        }
      }
      const float mean = sum_xor32(s) * (1.0f / D);
      float q = 0.f;
#pragma unroll
      for (int kk = 0; kk < KD; ++kk)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float t = xv[kk][e] - mean;
          q += t * t;
        }
      const float rstd = rsqrtf(sum_xor32(q) * (1.0f / D) + eps);
      if (aff1) {
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
          float gv[8], bv[8];
          load8(gamma1 + 16 * kk + 8 * g, gv);
          load8(beta1 + 16 * kk + 8 * g, bv);
#pragma unroll
          for (int e = 0; e < 8; ++e) hB[kk][e] = (f16)((xv[kk][e] - mean) * rstd * gv[e] + bv[e]);
        }
      } else {  // no elementwise affine (folded into W_qkv / b_qkv by the caller)
#pragma unroll
        for (int kk = 0; kk < KD; ++kk)
#pragma unroll
          for (int e = 0; e < 8; ++e) hB[kk][e] = (f16)((xv[kk][e] - mean) * rstd);
      }
    }

    // Attention output of every head as fp16 B operands of out^T = W_o ctx^T:
    // k-step ks of d_model covers head ks / KSH.
    f16x8 cB[KD];

#pragma unroll
    for (int j = 0; j < NH; ++j) {
      __builtin_amdgcn_sched_barrier(0);  // keep heads from interleaving (register pressure)
      // ---- projections of this wave's 32 tokens for head j ----------------------
      f16x8 qB[KSH];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int d0 = j * HD + dt * 32;
        // The biases start the accumulators (C operand of the first product).
        f32x16 qa, ka, va;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          const f32x4 tq = *reinterpret_cast<const f32x4*>(bias_qkv + d0 + 8 * qd + 4 * g);
          const f32x4 tk = *reinterpret_cast<const f32x4*>(bias_qkv + D + d0 + 8 * qd + 4 * g);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            qa[4 * qd + e] = tq[e];
            ka[4 * qd + e] = tk[e];
          }
        }
        const float bvl = bias_qkv[2 * D + d0 + li];
#pragma unroll
        for (int r = 0; r < 16; ++r) va[r] = bvl;
        const f16x8* wq = Wl + (d0 / 32) * KD * 64 + lane;
        const f16x8* wk = wq + (D / 32) * KD * 64;
        const f16x8* wv = wk + (D / 32) * KD * 64;
#pragma unroll
        for (int kk = 0; kk < KD; ++kk) {
          const f16x8 aq = wq[kk * 64];
          const f16x8 ak = wk[kk * 64];
          const f16x8 bv = wv[kk * 64];
          qa = mfma32x32x16(aq, hB[kk], qa);
          ka = mfma32x32x16(ak, hB[kk], ka);
          va = mfma32x32x16(hB[kk], bv, va);
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          qB[2 * dt + half] = acc_f16(qa, half);
          Kl[(w * KSH + 2 * dt + half) * 64 + lane] = acc_f16(ka, half);
          Vl[((w * NDT + dt) * 2 + half) * 64 + lane] = acc_f16(va, half);
        }
      }
      __syncthreads();

      // ---- S^T = K Q^T for all (at most 128) keys, one exact softmax pass (no
      // running max, no rescale), O^T = V^T P^T.
      // Every key tile is computed, branch-free: all four waves always write their
      // K/V slots (finite values, also past S), and masked keys get p = 0.  The
      // wasted tiles cost no latency -- the slowest wave bounds every barrier.
      f32x16 sacc[MAXT];
      float mx = kNegInf;
#pragma unroll
      for (int t = 0; t < MAXT; ++t) {
        sacc[t] = zero16();
#pragma unroll
        for (int ks = 0; ks < KSH; ++ks) sacc[t] = mfma32x32x16(Kl[(t * KSH + ks) * 64 + lane], qB[ks], sacc[t]);
        // Keys past S (last tile) and keys after the query (diagonal and later
        // tiles).  The bound is made opaque per head so that the 16 per-register
        // lane masks are formed here rather than hoisted (and spilled) across loops.
        if (32 * t + 32 > S || (CAUSAL && t >= w)) {
          int lim = S - 32 * t - 4 * g + opaque_zero();  // valid: offset < lim
          if (CAUSAL) lim = min(lim, tok - 32 * t - 4 * g + 1);
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
      // Unmasked, key 0 is valid for every query (finite max); a query whose keys
      // are all padded gets max -inf, all-zero probabilities and a zero row.
      float m = mx * c2;
      if constexpr (MASKED) m = mx == kNegInf ? 0.f : m;
      f32x16 ot[NDT];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) ot[dt] = zero16();
      float lp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < MAXT; ++t) {
        f16x8 pB[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) pB[r >> 3][r & 7] = (f16)__builtin_amdgcn_exp2f(fmaf(sacc[t][r], c2, -m));
        add_probs(pB[0], lp[0], lp[1]);
        add_probs(pB[1], lp[2], lp[3]);
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
            ot[dt] = mfma32x32x16(Vl[((t * NDT + dt) * 2 + half) * 64 + lane], pB[half], ot[dt]);
      }
      const float l = sum_xor32((lp[0] + lp[1]) + (lp[2] + lp[3]));
      // A query with no valid key (only a padded one) gets a zero row.
      const float inv = MASKED ? (l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f) : __builtin_amdgcn_rcpf(l);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int half = 0; half < 2; ++half) cB[j * KSH + 2 * dt + half] = scaled_f16(ot[dt], half, inv);
      __syncthreads();  // K/V of head j are dead; the next head may overwrite them
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- this sequence's residual, from the LN1 input still in registers: lane
    // (tok, g) holds columns 16kk + 8g + {0..7}; the out-projection layout wants
    // 32nt + 8qd + 4g + {0..3}, whose other half sits in the partner lane (tok, 1 - g).
    // Rows past S (and groups past the batch) were loaded as zeros.
    Raw4 xres[NNT][4];
#pragma unroll
    for (int kk = 0; kk < KD; ++kk) {
      // lane g = 0 keeps columns +0..3 and takes +8..11 from its partner; g = 1 takes
      // +4..7 and keeps +12..15
      Raw4 lo = {xpre[kk][0], xpre[kk][1], xpre[kk][2], xpre[kk][3]};
      Raw4 hi = {xpre[kk][4], xpre[kk][5], xpre[kk][6], xpre[kk][7]};
      const int nt = kk / 2, j = kk % 2;  // columns 16kk.. = tile nt, qd 2j and 2j + 1
      if constexpr (L::PARAMS) {
        swap_halves(lo, hi);
        xres[nt][2 * j] = lo;
        xres[nt][2 * j + 1] = hi;
      } else {  // (see the y exchange below)
        const Raw4 recv = partner_value(g ? lo : hi);
        xres[nt][2 * j] = g ? recv : lo;
        xres[nt][2 * j + 1] = g ? hi : recv;
      }
    }
    // ---- prefetch: the next sequence's LN1 input --------------------------------------
    load_ln1_input((sg + (int)gridDim.x) * G + grp);

    // ---- out^T = W_o ctx^T over all heads, started from b_o ---------------------------
    f32x16 oacc[NNT];  // lane (tok, g), reg r -> column 32nt + 8(r/4) + 4g + r%4
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const f32x4 bb = *reinterpret_cast<const f32x4*>(bias_o + 32 * nt + 8 * qd + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) oacc[nt][4 * qd + e] = bb[e];
      }
#pragma unroll
    for (int ks = 0; ks < KD; ++ks)
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt) oacc[nt] = mfma32x32x16(Wol[(nt * KD + ks) * 64 + lane], cB[ks], oacc[nt]);

    // ---- r = out + b_o + x;  y = LN2(r) ------------------------------------------
    float v[NNT][4][4];
    float s = 0.f;
    // A padded token's attention output is zero (masked_fill before the residual add).
    const bool tv = !MASKED || kbits.valid(tok);
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[nt][qd][e] = (tv ? oacc[nt][4 * qd + e] : 0.f) + (float)xres[nt][qd][e];
          s += v[nt][qd][e];
        }
    const float mean = sum_xor32(s) * (1.0f / D);
    float q = 0.f;
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float t = v[nt][qd][e] - mean;
          q += t * t;
        }
    const float rstd = rsqrtf(sum_xor32(q) * (1.0f / D) + eps);
    float o[NNT][4][4];
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int n0 = 32 * nt + 8 * qd + 4 * g;
        const f32x4 gg = *reinterpret_cast<const f32x4*>(gamma2 + n0);
        const f32x4 bb = *reinterpret_cast<const f32x4*>(beta2 + n0);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[nt][qd][e] = (v[nt][qd][e] - mean) * rstd * gg[e] + bb[e];
      }
    // fp16 rows leave as 16-byte pieces: for each pair of quads (qd = 2p, 2p + 1)
    // lane g = 0 collects columns 32nt + 16p + {0..7} and lane g = 1 columns
    // 32nt + 16p + 8 + {0..7}, one exchange with the partner lane each.
    if constexpr (sizeof(TX) == 2) {
      f16x8 yo[NNT][2];
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          f16x4 h0, h1;  // this lane's quads 2pr and 2pr + 1
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            h0[e] = (f16)o[nt][2 * pr][e];
            h1[e] = (f16)o[nt][2 * pr + 1][e];
          }
          if constexpr (L::PARAMS) {
            swap_halves(h0, h1);  // g = 0: both lanes' quad 2pr; g = 1: both lanes' quad 2pr + 1
          } else {
            // Parameters read from global memory (no LDS left for them): with the
            // select-based exchanges here and for the residual above, the compiler's
            // schedule of the gamma2 / beta2 loads measured ~8 % faster (head_dim 64).
            const f16x4 recv = partner_value(g ? h0 : h1);
            const f16x4 a = g ? recv : h0, b = g ? h1 : recv;
            h0 = a;
            h1 = b;
          }
          yo[nt][pr] = f16x8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
        }
      if (tok_ok && live) {
        TX* yrow = y + row * D;
#pragma unroll
        for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
          for (int pr = 0; pr < 2; ++pr) *reinterpret_cast<f16x8*>(yrow + 32 * nt + 16 * pr + 8 * g) = yo[nt][pr];
      }
    } else {
      if (tok_ok && live) {
        TX* yrow = y + row * D;
#pragma unroll
        for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
          for (int qd = 0; qd < 4; ++qd) store4(yrow + 32 * nt + 8 * qd + 4 * g, o[nt][qd]);
      }
    }
    if (!FULL && resid_out && tok_ok && live) {
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) store4(resid_out + row * D + 32 * nt + 8 * qd + 4 * g, v[nt][qd]);
    }
    if constexpr (FULL) {
      wait_vmcnt<2 * NNT>();  // the prefetch, not the stores behind it
      input_complete();
    }
  }  // sequence loop
}

bool layer_small_ok(int64_t seq_len, int64_t d_model, int64_t heads) {
  if (heads <= 0 || d_model % heads != 0) return false;
  const int64_t hd = d_model / heads;
  const bool shape = (d_model == 128 && (hd == 32 || hd == 64)) || (d_model == 64 && (hd == 32 || hd == 64)) ||
                     (d_model == 96 && hd == 32);
  return shape && seq_len >= 1 && seq_len <= kSmallMaxS;
}

// Persistent grid: one workgroup per CU (the staged weights fill most of the
// LDS), each walking the batch with stride gridDim.x.

// Always four waves: the waves past the sequence's last 32-token tile still
// share the weight staging (and compute masked tiles nobody reads).
template <int D, int HD, bool CAUSAL, typename TX, int G, bool FULL>
static hipError_t launch_small_kernel(const SmallLayerArgs& a, float c2, int64_t grid) {
  if (a.valid_mask)
    hipLaunchKernelGGL((layer_small_kernel<D, HD, CAUSAL, true, TX, G, FULL>), dim3((unsigned)grid),
                       dim3(64 * kSmallWaves * G), 0, a.stream, static_cast<const TX*>(a.x),
                       static_cast<const f16*>(a.w_qkv), a.b_qkv, static_cast<const f16*>(a.w_o), a.b_o, a.ln1_w,
                       a.ln1_b, a.ln2_w, a.ln2_b, static_cast<TX*>(a.y), a.resid_out, (int)a.batch, (int)a.seq_len,
                       c2, a.eps, a.valid_mask);
  else
    hipLaunchKernelGGL((layer_small_kernel<D, HD, CAUSAL, false, TX, G, FULL>), dim3((unsigned)grid),
                       dim3(64 * kSmallWaves * G), 0, a.stream, static_cast<const TX*>(a.x),
                       static_cast<const f16*>(a.w_qkv), a.b_qkv, static_cast<const f16*>(a.w_o), a.b_o, a.ln1_w,
                       a.ln1_b, a.ln2_w, a.ln2_b, static_cast<TX*>(a.y), a.resid_out, (int)a.batch, (int)a.seq_len,
                       c2, a.eps, nullptr);
  return hipGetLastError();
}

template <int D, int HD, bool CAUSAL, typename TX>
static hipError_t launch_small(const SmallLayerArgs& a, float c2) {
  constexpr int G = small_groups<D, HD, TX>();
  const int64_t groups = (a.batch + G - 1) / G;
  const int64_t grid = groups < compute_units() ? groups : compute_units();
  if constexpr (G == 1 && sizeof(TX) == 2) {
    if (a.seq_len == 32 * kSmallWaves && !a.resid_out) return launch_small_kernel<D, HD, CAUSAL, TX, G, true>(a, c2, grid);
  }
  return launch_small_kernel<D, HD, CAUSAL, TX, G, false>(a, c2, grid);
}

template <int D, int HD, bool CAUSAL>
static hipError_t small_dtype(const SmallLayerArgs& a, float c2) {
  return a.x_dtype == kF16 ? launch_small<D, HD, CAUSAL, f16>(a, c2) : launch_small<D, HD, CAUSAL, float>(a, c2);
}

template <bool CAUSAL>
static hipError_t small_shape(const SmallLayerArgs& a, float c2) {
  const int64_t hd = a.d_model / a.heads;
  if (a.d_model == 128) {
    if (hd == 32) return small_dtype<128, 32, CAUSAL>(a, c2);
    return small_dtype<128, 64, CAUSAL>(a, c2);
  }
  if (a.d_model == 64) {
    if (hd == 32) return small_dtype<64, 32, CAUSAL>(a, c2);
    return small_dtype<64, 64, CAUSAL>(a, c2);
  }
  return small_dtype<96, 32, CAUSAL>(a, c2);
}

bool layer_fused_ok(int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int x_dtype) {
  if (x_dtype != kF16 && x_dtype != kF32) return false;
  return layer_small_ok(seq_len, d_model, heads) ||
         (layer_split_ok(seq_len, d_model, heads) && layer_split_pays(batch, seq_len, d_model, x_dtype));
}

hipError_t run_layer_small(const SmallLayerArgs& a) {
  if (a.batch < 0 || a.batch > 0x7fffffff || !layer_fused_ok(a.batch, a.seq_len, a.d_model, a.heads, a.x_dtype))
    return hipErrorInvalidValue;
  if (a.batch == 0) return hipSuccess;
  if (layer_split_takes(a)) return run_layer_split(a);
  const double hd = (double)(a.d_model / a.heads);
  const float c2 = (float)(1.0 / sqrt(hd)) * 1.4426950408889634f;
  return a.causal ? small_shape<true>(a, c2) : small_shape<false>(a, c2);
}

}  // namespace cobra
