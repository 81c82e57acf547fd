// Flash-style multi-head attention over a packed qkv buffer, causal or not.
//
// Replaces the reference's _attn_kernel / _attn_cfgs / _tl_attn
// (torch_transformer_benchmark.py:572-649, 788-854), which is causal-only, and
// the SDPA call the reference uses for non-causal attention (TTB:1240-1253).
// Semantics per query row i (TTB:98-113): s_j = (q_i . k_j) * scale, masked
// keys (j > i under causality, j >= S) are -inf, p = softmax(s) in fp32,
// ctx_i = sum_j p_j v_j.  The [S, S] score matrix is never formed: keys are
// visited in blocks with an online (running max / running sum) softmax in the
// exp2 domain, normalised once at the end.  An optional key mask (the
// reference's valid_token_mask, TTB:106-109) arrives as packed bits, one
// 64-bit word per 64 keys of a sequence, produced from the [B, S] byte mask by
// mask_bits_kernel; a query with no valid key gets a zero context row.
//
// CDNA4 mapping (one wave = 32 queries, v_mfma_f32_32x32x16_f16):
//   * scores are computed transposed, S^T = K . Q^T, so the C layout gives
//     every lane ONE query (col = lane % 32) and 16 keys of a 32-key tile;
//     the running max, running sum and rescale of that query stay in the lane
//     (plus one exchange with lane ^ 32, which holds the other 16 keys);
//   * the output is accumulated transposed as well, O^T += V^T . P^T.  The
//     probabilities of a 16-key step already sit in the lane in the B-operand
//     position (col = query); their key order is the C layout's row order
//     {4g..4g+3, 8+4g..8+4g+3} (g = lane / 32).  V stays row-major in LDS and
//     the V^T operand is read in exactly that key order with two
//     ds_read_b64_tr_b16 (a 4x4 transpose within each 16-lane group);
//   * K and V tiles are row-major in LDS, 16-byte chunks XOR-swizzled by row
//     (no padding, conflict-free operand reads), filled by coalesced LDS-DMA
//     (global_load_lds_dwordx4, 1 KB per wave instruction) 3-4 key blocks ahead:
//     each wave waits for its own transfers (vmcnt), one barrier per block
//     publishes them and retires the stage the next DMA refills;
//   * the Q tile arrives the same way (its own LDS region in short-sequence
//     launches, so it overlaps the first K/V stages), and the output tile leaves
//     through LDS so that the stores to ctx are whole coalesced rows;
//   * the Q fragments are pre-scaled by scale * log2(e) and each score tile's
//     accumulator starts at -m (the query's running max), so the matrix cores
//     deliver s - m in the exp2 domain and p = exp2 of the accumulator;
//   * no block maximum in the common case: once a wave's queries have a
//     running max (block 0), a block's probabilities are formed against it
//     directly and accepted if every lane's block sum is <= 2^16 (so every
//     probability is, well inside fp16); a block that fails the check -- a
//     score ~10-16 above the running max -- forms its scores again and takes
//     the max path: the running max then moves (rescaling O and the sum) only
//     when the block raises it by more than 2^8, and the whole wave skips the
//     rescale when no lane needs it;
//   * the running sum adds the fp16 probabilities the P.V product consumes
//     (v_dot2_f32_f16 against ones, fp32 accumulation), and the max/sum
//     exchange with lane ^ 32 uses v_permlane32_swap;
//   * key masks: the block's validity word is a scalar load (it waits in
//     lgkmcnt, never behind the K/V transfers in vmcnt); a block without a
//     valid key is skipped by the whole workgroup, a fully valid one costs a
//     compare, and only partly valid blocks mask per key.
// q, k, v and ctx are fp16 or bf16 (a template type): the bf16 form uses
// v_mfma_f32_32x32x16_bf16 and v_dot2_f32_bf16 and rounds the probabilities to
// bf16, everything else is the same code.
#include "common.hpp"
#include "kernels.hpp"
#include "lds_dma.hpp"

namespace cobra {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ typename Op16<T>::V4 lds_read_tr16(const T* p) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  return __builtin_bit_cast(typename Op16<T>::V4, r);
}

// Chunk swizzle of a [rows][HD] fp16 tile: 16-byte chunk c of row r lives at
// chunk c ^ swz(r).  Chosen so that both LDS read patterns are conflict-free:
// the K operand (16 consecutive rows, one chunk each) and the V^T transpose
// read (4 consecutive rows x 4 consecutive chunks per 32 lanes).
template <int HD>
__device__ __forceinline__ int swz(int row) {
  if constexpr (HD == 16) {
    return (row >> 3) & 1;  // 8 rows per 256 bytes
  } else if constexpr (HD == 32) {
    return (row >> 2) & 3;  // 4 rows per 256 bytes
  } else if constexpr (HD == 64) {
    const int p = (row >> 1) & 7;     // row pair (2 rows per 256 bytes)
    return ((p & 1) << 2) | (p >> 1);  // consecutive pairs differ in the 4-chunk group
  } else {
    const int r = row & 15;            // >= 256-byte rows
    return ((r & 3) << 2) | (r >> 2);  // 4 consecutive rows in 4 distinct 4-chunk groups
  }
}

constexpr float kLazyRescale = 8.0f;  // log2 units
constexpr float kAcceptSum = 65536.0f;  // a lane's tile sum accepted without a block max

__device__ __forceinline__ f32x16 splat16(float v) {
  f32x16 r;
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = v;
  return r;
}

}  // namespace

template <int HD, int NW, int BN, int ST, bool CAUSAL, bool MASKED, typename TQ>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(const TQ* __restrict__ qkv, TQ* __restrict__ ctx,
                                                           int S, int H, int hd, float c2, int nqb,
                                                           const uint64_t* __restrict__ key_bits, int nwords) {
  using V8 = typename Op16<TQ>::V8;
  using V4 = typename Op16<TQ>::V4;
  using V2 = typename Op16<TQ>::V2;
  constexpr int BM = 32 * NW;          // queries per workgroup
  constexpr int KS = HD / 16;          // k-steps of the QK^T product
  constexpr int ND = (HD + 31) / 32;   // 32-row blocks of d in O^T
  constexpr int NT = NW * 64;
  constexpr int CPR = HD / 8;          // 16-byte chunks per row
  constexpr int TB = BN * HD * 2;      // bytes of one K (or V) tile
  constexpr int SB = 2 * TB;           // bytes of one stage: K tile, then V tile
  constexpr int NI = SB / 1024;        // 1 KB DMA spans per stage
  constexpr int LPT = NI / NW;         // spans per wave per stage
  constexpr int QPT = BM * HD * 2 / 1024 / NW;  // Q-tile spans per wave
  static_assert(HD % 16 == 0 && BN % 32 == 0, "tile geometry");
  static_assert(BN == 32 || BN == 64 || BN == 128, "key-mask words");
  constexpr int KW = BN > 64 ? 2 : 1;  // validity words per key block
  static_assert(NI % NW == 0 && LPT >= 1 && (NI / 2) % 1 == 0, "every wave DMAs whole spans of each stage");
  // Short-sequence launches (<= 4 waves) give the Q tile its own LDS region, so its
  // DMA overlaps the first K/V stages instead of preceding them; 8-wave launches
  // (long sequences) stage it through the K/V stages to keep LDS small.
  constexpr bool QSEP = NW <= 4;
  constexpr int QB = BM * HD * 2;
  constexpr int LDSB = ST * SB + (QSEP ? QB : 0);
  static_assert(BM * HD * 2 <= ST * SB, "the output tile passes through the K/V stages");
  static_assert(ST >= 2 && (ST - 1) * LPT < 64, "vmcnt range");
  static_assert(LDSB <= 163840, "LDS budget");

  __shared__ __attribute__((aligned(1024))) char smem[LDSB];
  char* const qtile = smem + (QSEP ? ST * SB : 0);

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int qb = id % nqb;
  const int bh = id / nqb;
  const int h = bh % H;
  const int64_t b = bh / H;
  const int D = H * hd;
  const int64_t ld = 3 * (int64_t)D;
  const TQ* qbase = qkv + b * S * ld + h * hd;
  const TQ* kbase = qbase + D;
  const TQ* vbase = qbase + 2 * D;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, li = lane & 31;
  const int q0w = qb * BM + w * 32;  // this wave's first query
  const int qi = q0w + li;           // this lane's query

  // Row-major [rows][HD] tiles in LDS, chunk c of row r at c ^ swz(r), filled by
  // coalesced LDS-DMA: 1 KB span `sp` of a tile holds rows sp*1024/(2HD) ..; each lane
  // fetches the global chunk that belongs in its slot.  Rows past S fetch row S-1 and
  // chunks past hd fetch chunk 0 (finite values; masked, zero-weighted or not stored).
  auto dma_tile = [&](char* tile, int sp, const TQ* base, int row0) {
    const int o = sp * 1024 + 16 * lane;
    const int row = o / (2 * HD), pos = (o % (2 * HD)) / 16;
    const int r = min(row0 + row, S - 1);
    const int d0 = 8 * (pos ^ swz<HD>(row));
    dma16(base + (int64_t)r * ld + (d0 < hd ? d0 : 0), tile + sp * 1024);
  };

  // Q^T fragments: B operand of S^T = K . Q^T (k = d), staged through LDS and
  // pre-scaled by scale * log2(e) so that the products come out in the exp2 domain.
#pragma unroll
  for (int i = 0; i < QPT; ++i) dma_tile(qtile, w + NW * i, qbase, qb * BM);

  // K/V stages: ST tiles deep, one barrier per key block.  A block that lies wholly
  // inside the sequence needs no row clamp, so its sources are this lane's fixed
  // pointers (row and chunk within the tile, K or V) plus the block's wave-uniform
  // offset: no per-block 64-bit address arithmetic on the vector ALU.  The block
  // reaching past S takes the clamped path.
  const TQ* kv_src[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int span = w + NW * i;
    const bool v = span >= NI / 2;
    const int o = (v ? span - NI / 2 : span) * 1024 + 16 * lane;
    const int row = o / (2 * HD), pos = (o % (2 * HD)) / 16;
    const int d0 = 8 * (pos ^ swz<HD>(row));
    kv_src[i] = (v ? vbase : kbase) + (int64_t)row * ld + (d0 < hd ? d0 : 0);
  }
  auto issue = [&](int stage, int kb) {
    char* sbase = smem + stage * SB;
    if (kb + BN <= S) {
      const int64_t step = (int64_t)kb * ld;
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const int span = w + NW * i;
        const bool v = span >= NI / 2;
        dma16(kv_src[i] + step, sbase + (v ? TB : 0) + (v ? span - NI / 2 : span) * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const int span = w + NW * i;
        const bool v = span >= NI / 2;
        dma_tile(sbase + (v ? TB : 0), v ? span - NI / 2 : span, v ? vbase : kbase, kb);
      }
    }
  };

  f32x16 o[ND];
#pragma unroll
  for (int j = 0; j < ND; ++j) o[j] = zero16();
  float m_run = 0.f;  // running max in the exp2 domain, set by block 0
  float l_run = 0.f;  // this lane's share of the running sum
  bool started = false;  // key masks: the running max is set by the first block with a valid key
  const uint64_t* krow = MASKED ? key_bits + b * nwords : nullptr;
  const V2 ones = {(TQ)1.0f, (TQ)1.0f};

  // Per-lane V^T read geometry (see the header): row within a 16-key step,
  // column within a 32-wide d tile.
  const int vr = 4 * g + ((lane & 15) >> 2);
  const int vc = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  const int kend = CAUSAL ? min(S, (qb + 1) * BM) : S;
  const int nblk = (kend + BN - 1) / BN;
  const int pre = min(ST - 1, nblk);  // key blocks in flight before the loop
  if constexpr (QSEP) {
#pragma unroll
    for (int s = 0; s < ST - 1; ++s)
      if (s < nblk) issue(s, s * BN);
    // The Q tile is the oldest transfer: wait for it alone.
    if constexpr (ST >= 4) {
      if (pre >= 3) {
        wait_vmcnt<3 * LPT>();
      } else if (pre == 2) {
        wait_vmcnt<2 * LPT>();
      } else {
        wait_vmcnt<LPT>();
      }
    } else {
      if (pre >= 2) {
        wait_vmcnt<2 * LPT>();
      } else {
        wait_vmcnt<LPT>();
      }
    }
  } else {
    wait_vmcnt<0>();
  }
  stage_barrier();
  V8 qf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int row = w * 32 + li, d0 = kk * 16 + g * 8;
    const V8 q = *reinterpret_cast<const V8*>(qtile + row * 2 * HD + 16 * ((2 * kk + g) ^ swz<HD>(row)));
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[kk][e] = d0 < hd ? (TQ)((float)q[e] * c2) : (TQ)0.0f;
  }
  if constexpr (!QSEP) {
    lds_barrier();  // every wave has its Q fragments before the stages are refilled
#pragma unroll
    for (int s = 0; s < ST - 1; ++s)
      if (s < nblk) issue(s, s * BN);
  }
  for (int n = 0; n < nblk; ++n) {
    const int kb = n * BN;
    // Key-validity bits of keys kb .. kb+BN-1 (bit j = key kb + j); the scalar
    // load completes under the barrier's lgkmcnt wait below.
    uint64_t kw[KW];
    if constexpr (MASKED) {
      const int w0 = kb >> 6;
      if constexpr (BN == 128) {
        kw[0] = krow[w0];
        kw[1] = krow[min(w0 + 1, nwords - 1)];
        if (w0 + 1 >= nwords) kw[1] = 0;
      } else if constexpr (BN == 64) {
        kw[0] = krow[w0];
      } else {
        kw[0] = (krow[w0] >> (kb & 32)) & 0xffffffffull;
      }
    }
    // Blocks n+1 .. n+ST-2 may still be in flight; block n must have landed.
    const int ahead = min(ST - 2, nblk - 1 - n);
    if constexpr (ST >= 4) {
      if (ahead >= 2) {
        wait_vmcnt<2 * LPT>();
      } else if (ahead == 1) {
        wait_vmcnt<LPT>();
      } else {
        wait_vmcnt<0>();
      }
    } else if constexpr (ST == 3) {
      if (ahead >= 1) {
        wait_vmcnt<LPT>();
      } else {
        wait_vmcnt<0>();
      }
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();  // block n visible to all waves; every wave is done with block n-1
    if (n + ST - 1 < nblk) issue((n + ST - 1) % ST, (n + ST - 1) * BN);
    bool kpart = false;  // some key of the block is padded
    if constexpr (MASKED) {
      constexpr uint64_t kFull = BN == 32 ? 0xffffffffull : ~0ull;
      uint64_t any = 0, all = kFull;
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        any |= kw[k];
        all &= kw[k];
      }
      if (any == 0) continue;  // no valid key: the block adds nothing (uniform over the workgroup)
      kpart = all != kFull;
    }
    const TQ* Kc = reinterpret_cast<const TQ*>(smem + (n % ST) * SB);
    const TQ* Vc = reinterpret_cast<const TQ*>(smem + (n % ST) * SB + TB);
    // s = scores in the exp2 domain minus the running max: the accumulator
    // starts at -m_run (every register of a lane belongs to the lane's query).
    // Masks only where a block reaches past S, causally past this wave's first
    // query, or holds a padded key.
    const bool need_mask = kb + BN > S || (CAUSAL && kb + BN > q0w + 1) || kpart;
    auto scores = [&](f32x16(&s)[BN / 32]) {
#pragma unroll
      for (int t = 0; t < BN / 32; ++t) {
        s[t] = splat16(-m_run);
        const int row = t * 32 + li;
        const TQ* kr = Kc + row * HD;
        const int sw = swz<HD>(row);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const V8 a = *reinterpret_cast<const V8*>(kr + (((2 * kk + g) ^ sw) * 8));
          s[t] = mfma32x32x16(a, qf[kk], s[t]);
        }
      }
      if (need_mask) {
        // Register r of tile t holds key kb + 4g + kc with kc = 32t + 8(r/4) + r%4,
        // a constant: the key is past S or causally after the query iff kc > lim.
        // A tile whose keys are all live for every lane of the wave is skipped
        // (a uniform branch per tile, which also keeps the predicates of one tile
        // at a time in scalar registers).
        const int lim = CAUSAL ? min(S - 1, qi) - kb - 4 * g : S - 1 - kb - 4 * g;
        uint64_t lw[KW];  // this lane's view: bit c = key kb + 32*(word half) + 4g + c
#pragma unroll
        for (int k = 0; k < KW; ++k) lw[k] = MASKED ? kw[k] >> (4 * g) : 0;
#pragma unroll
        for (int t = 0; t < BN / 32; ++t) {
          const uint32_t tw = MASKED ? (uint32_t)(lw[t >> 1] >> ((t & 1) * 32)) : 0u;
          bool part = t * 32 + 27 > lim;  // the tile's last key for this lane: kc = 32t + 27
          if constexpr (MASKED) part = part || (tw & 0x0F0F0F0Fu) != 0x0F0F0F0Fu;
          if (__builtin_amdgcn_ballot_w64(part)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int kc = t * 32 + 8 * (r >> 2) + (r & 3);
              bool dead = kc > lim;
              if constexpr (MASKED) dead = dead || !((tw >> (8 * (r >> 2) + (r & 3))) & 1);
              if (dead) s[t][r] = kNegInf;
            }
          }
        }
      }
    };
    // The running max moves (rescaling O and the sum, and the scores still to be
    // exponentiated: tiles t0 ..) only when the wave's max over those scores is
    // more than kLazyRescale above it; block 0 (or, with key masks, the first
    // block with a valid key for the query) sets it.
    auto rescale = [&](f32x16(&s)[BN / 32], int t0, bool first) {
      float mx = kNegInf;
#pragma unroll
      for (int t = 0; t < BN / 32; ++t)
        if (t >= t0)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
      mx = max_xor32(mx);  // relative to m_run
      if constexpr (MASKED) {
        const bool live = mx != kNegInf;
        if (__builtin_amdgcn_ballot_w64(started ? mx > kLazyRescale : live)) {
          const float inc = started ? fmaxf(mx, 0.f) : (live ? mx : 0.f);
          const float alpha = started ? __builtin_amdgcn_exp2f(-inc) : 1.f;
          l_run *= alpha;
#pragma unroll
          for (int j = 0; j < ND; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
#pragma unroll
          for (int t = 0; t < BN / 32; ++t)
            if (t >= t0)
#pragma unroll
              for (int r = 0; r < 16; ++r) s[t][r] -= inc;
          m_run += inc;
          started = started || live;
        }
      } else if (first || __builtin_amdgcn_ballot_w64(mx > kLazyRescale)) {
        // Block 0 holds key 0, valid for every query, so its mx is finite.
        const float inc = first ? mx : fmaxf(mx, 0.f);
        if (!first) {
          const float alpha = __builtin_amdgcn_exp2f(-inc);
          l_run *= alpha;
#pragma unroll
          for (int j = 0; j < ND; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
        }
#pragma unroll
        for (int t = 0; t < BN / 32; ++t)
          if (t >= t0)
#pragma unroll
            for (int r = 0; r < 16; ++r) s[t][r] -= inc;
        m_run += inc;
      }
    };

    f32x16 s[BN / 32];
    scores(s);
    // Once every query of the wave has a running max, no block maximum is formed:
    // each 32-key tile's probabilities are taken against the running max directly
    // and accepted when every lane's tile sum is at most 2^16, so that no
    // probability exceeds 2^16 (fp16 holds each one; an fp16 overflow reads as an
    // infinite sum) and the fp32 sums and products stay far from overflow.  A
    // tile that fails the check -- a score more than ~12-16 above the running
    // max, rare after the first block -- rescales over the block's remaining
    // tiles and is exponentiated again.  Tile by tile, the P.V products of one
    // tile overlap the exponentials of the next.
    const bool direct = MASKED ? !__builtin_amdgcn_ballot_w64(!started) : n != 0;
    if (!direct) rescale(s, 0, !MASKED);
#pragma unroll
    for (int t = 0; t < BN / 32; ++t) {
      // p = exp2(s) rounded to the operand type, in the P.V B-operand layout (two
      // 16-key steps), and this lane's share of the tile's row sum over those
      // rounded values (the ones the P.V product uses), fp32 accumulation.
      V8 pf[2];
      float lt;
      auto probs = [&]() {
#pragma unroll
        for (int r = 0; r < 16; ++r) pf[r >> 3][r & 7] = (TQ)__builtin_amdgcn_exp2f(s[t][r]);
        lt = 0.f;
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const V2 pr = {pf[k][2 * e], pf[k][2 * e + 1]};
            lt = dot2(pr, ones, lt);
          }
      };
      probs();
      if (direct && __builtin_amdgcn_ballot_w64(!(lt <= kAcceptSum))) {
        rescale(s, t, false);
        probs();
      }
      l_run += lt;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const int ks = 2 * t + kh;
#pragma unroll
        for (int j = 0; j < ND; ++j) {
          V4 lo, hi;
          if (HD >= 32 || vc < HD) {
            const int c = j * 32 + vc;
            const int r0 = ks * 16 + vr, r1 = r0 + 8;
            lo = lds_read_tr16(Vc + r0 * HD + (((c >> 3) ^ swz<HD>(r0)) * 8) + (c & 7));
            hi = lds_read_tr16(Vc + r1 * HD + (((c >> 3) ^ swz<HD>(r1)) * 8) + (c & 7));
          } else {
            lo = hi = V4{(TQ)0.0f, (TQ)0.0f, (TQ)0.0f, (TQ)0.0f};  // d beyond a 16-wide head
          }
          const V8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[j] = mfma32x32x16(a, pf[kh], o[j]);
        }
      }
    }
  }

  // Output through LDS: O^T quads into [BM][HD] rows, then whole 16-byte chunks per
  // lane, so the stores to ctx are row-contiguous.
  const float l_tot = sum_xor32(l_run);
  const float inv = MASKED ? (l_tot > 0.f ? 1.0f / l_tot : 0.f) : 1.0f / l_tot;
  lds_barrier();  // every wave is done with the last stage
#pragma unroll
  for (int j = 0; j < ND; ++j)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = j * 32 + 8 * q4 + 4 * g;
      if (HD >= 32 || d < HD) {
        const int row = w * 32 + li;
        V4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (TQ)(o[j][q4 * 4 + e] * inv);
        *reinterpret_cast<V4*>(smem + row * 2 * HD + 16 * ((d >> 3) ^ swz<HD>(row)) + 8 * g) = v;
      }
    }
  lds_barrier();
  for (int idx = tid; idx < BM * CPR; idx += NT) {
    const int row = idx / CPR, c = idx % CPR;
    const int q = qb * BM + row, d0 = 8 * c;
    if (q < S && d0 < hd)
      *reinterpret_cast<V8*>(ctx + (b * S + q) * (int64_t)D + h * hd + d0) =
          *reinterpret_cast<const V8*>(smem + row * 2 * HD + 16 * (c ^ swz<HD>(row)));
  }
}

// Wide heads over short sequences (head_dim 128 / 256, S <= 128): one workgroup
// per (sequence, head), four waves of 32 queries, every key present at once, so
// the softmax is exact in one pass (no running max, no rescale, no per-block
// barrier).  LDS holds K [128][HD] and, in turn, the Q tile and then V [128][HD]
// (64 KB each at head_dim 256): V streams in while the scores and the softmax
// run.  Same fragment conventions as attn_fwd_kernel: S^T = K . Q^T with Q
// pre-scaled by scale * log2(e), O^T = V^T . P^T with V^T read by
// ds_read_b64_tr_b16.  Rows past S fetch row S-1 (finite; their keys are masked
// and their queries never stored).
template <int HD, bool CAUSAL, bool MASKED, typename TQ>
__global__ __launch_bounds__(256) void attn_short_kernel(const TQ* __restrict__ qkv, TQ* __restrict__ ctx, int S,
                                                         int H, float c2, const uint64_t* __restrict__ key_bits,
                                                         int nwords) {
  using V8 = typename Op16<TQ>::V8;
  using V4 = typename Op16<TQ>::V4;
  using V2 = typename Op16<TQ>::V2;
  constexpr int NW = 4, BM = 128;
  constexpr int KS = HD / 16, ND = HD / 32, CPR = HD / 8;
  constexpr int TB = BM * HD * 2;   // one [128][HD] tile
  constexpr int NI = TB / 1024;     // 1 KB spans per tile
  constexpr int LPT = NI / NW;      // spans per wave per tile
  static_assert(HD == 128 || HD == 256, "wide heads");
  static_assert(LPT >= 1 && LPT < 32, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[2 * TB];
  char* const ktile = smem;
  char* const qvtile = smem + TB;  // Q, then V

  const int bh = xcd_remap(blockIdx.x, gridDim.x);
  const int h = bh % H;
  const int64_t b = bh / H;
  const int D = H * HD;
  const int64_t ld = 3 * (int64_t)D;
  const TQ* qbase = qkv + b * S * ld + h * HD;
  const TQ* kbase = qbase + D;
  const TQ* vbase = qbase + 2 * D;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5, li = lane & 31;
  const int qi = w * 32 + li;  // this lane's query

  auto dma_tile = [&](char* tile, int sp, const TQ* base) {
    const int o = sp * 1024 + 16 * lane;
    const int row = o / (2 * HD), pos = (o % (2 * HD)) / 16;
    const int r = min(row, S - 1);
    dma16(base + (int64_t)r * ld + 8 * (pos ^ swz<HD>(row)), tile + sp * 1024);
  };
  // Q, then K (wave w: spans w, w + 4, ...); V follows once Q has been read.
#pragma unroll
  for (int i = 0; i < LPT; ++i) dma_tile(qvtile, w + NW * i, qbase);
#pragma unroll
  for (int i = 0; i < LPT; ++i) dma_tile(ktile, w + NW * i, kbase);
  // Key validity words (keys 0..63, 64..127; keys past S are dead anyway), as this
  // lane sees them: shifted by 4g, so that register r of key tile t tests the fixed
  // bit 32(t % 2) + 8(r / 4) + r % 4 of word t / 2.
  uint64_t lw0 = ~0ull, lw1 = ~0ull;
  if constexpr (MASKED) {
    lw0 = key_bits[b * nwords] >> (4 * g);
    lw1 = key_bits[b * nwords + min(1, nwords - 1)] >> (4 * g);
  }
  wait_vmcnt<LPT>();  // Q
  stage_barrier();
  V8 qf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const V8 q = *reinterpret_cast<const V8*>(qvtile + qi * 2 * HD + 16 * ((2 * kk + g) ^ swz<HD>(qi)));
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[kk][e] = (TQ)((float)q[e] * c2);
  }
  wait_vmcnt<0>();  // K
  lds_barrier();    // every wave has its Q fragments and sees the whole K tile
#pragma unroll
  for (int i = 0; i < LPT; ++i) dma_tile(qvtile, w + NW * i, vbase);

  const bool active = 32 * w < S;  // waves wholly past S only take part in the transfers and barriers
  f32x16 o[ND];
#pragma unroll
  for (int j = 0; j < ND; ++j) o[j] = zero16();
  float l = 0.f;
  V8 pf[8];
  if (active) {
    const int nkt = CAUSAL ? min((S + 31) / 32, w + 1) : (S + 31) / 32;  // key tiles with a live key
    f32x16 sacc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      sacc[t] = zero16();
      if (t < nkt) {
        const int row = t * 32 + li;
        const char* krow = ktile + row * 2 * HD;
        const int sw = swz<HD>(row);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
          sacc[t] = mfma32x32x16(*reinterpret_cast<const V8*>(krow + 16 * ((2 * kk + g) ^ sw)), qf[kk], sacc[t]);
      }
    }
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = t * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        bool dead = t >= nkt || key >= S || (CAUSAL && key > qi);
        if constexpr (MASKED) dead = dead || !(((t < 2 ? lw0 : lw1) >> (32 * (t & 1) + 8 * (r >> 2) + (r & 3))) & 1);
        if (dead) sacc[t][r] = kNegInf;
        mx = fmaxf(mx, sacc[t][r]);
      }
    mx = max_xor32(mx);
    // A query with no valid key (token masks) has max -inf: all-zero probabilities.
    const float m = mx == kNegInf ? 0.f : mx;
    const V2 ones = {(TQ)1.0f, (TQ)1.0f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) pf[2 * t + (r >> 3)][r & 7] = (TQ)__builtin_amdgcn_exp2f(sacc[t][r] - m);
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) l = dot2(V2{pf[k][2 * e], pf[k][2 * e + 1]}, ones, l);
  }
  wait_vmcnt<0>();  // V
  lds_barrier();
  if (active) {
    const int vr = 4 * g + ((lane & 15) >> 2);
    const int vc = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const TQ* Vc = reinterpret_cast<const TQ*>(qvtile);
    const int nks = CAUSAL ? 2 * min((S + 31) / 32, w + 1) : 2 * ((S + 31) / 32);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      if (ks < nks) {
#pragma unroll
        for (int j = 0; j < ND; ++j) {
          const int c = j * 32 + vc;
          const int r0 = ks * 16 + vr, r1 = r0 + 8;
          const V4 lo = lds_read_tr16(Vc + r0 * HD + (((c >> 3) ^ swz<HD>(r0)) * 8) + (c & 7));
          const V4 hi = lds_read_tr16(Vc + r1 * HD + (((c >> 3) ^ swz<HD>(r1)) * 8) + (c & 7));
          const V8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[j] = mfma32x32x16(a, pf[ks], o[j]);
        }
      }
    }
  }
  const float l_tot = sum_xor32(l);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  // Output through LDS (the K tile is dead): O^T quads into [128][HD] rows, then whole
  // 16-byte chunks per lane, so the stores to ctx are row-contiguous.
  lds_barrier();
  if (active) {
#pragma unroll
    for (int j = 0; j < ND; ++j)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = j * 32 + 8 * q4 + 4 * g;
        V4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (TQ)(o[j][q4 * 4 + e] * inv);
        *reinterpret_cast<V4*>(ktile + qi * 2 * HD + 16 * ((d >> 3) ^ swz<HD>(qi)) + 8 * g) = v;
      }
  }
  lds_barrier();
  for (int idx = threadIdx.x; idx < BM * CPR; idx += NW * 64) {
    const int row = idx / CPR, c = idx % CPR;
    if (row < S)
      *reinterpret_cast<V8*>(ctx + (b * S + row) * (int64_t)D + h * HD + 8 * c) =
          *reinterpret_cast<const V8*>(ktile + row * 2 * HD + 16 * (c ^ swz<HD>(row)));
  }
}

template <int HD, bool CAUSAL, typename TQ>
static hipError_t launch_attn_short(const AttnArgs& a, float c2) {
  const int64_t grid = (int64_t)a.heads * a.batch;
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  const int nwords = (int)mask_words(a.seq_len);
  if (a.key_bits)
    hipLaunchKernelGGL((attn_short_kernel<HD, CAUSAL, true, TQ>), dim3((unsigned)grid), dim3(256), 0, a.stream,
                       static_cast<const TQ*>(a.qkv), static_cast<TQ*>(a.ctx), a.seq_len, a.heads, c2, a.key_bits,
                       nwords);
  else
    hipLaunchKernelGGL((attn_short_kernel<HD, CAUSAL, false, TQ>), dim3((unsigned)grid), dim3(256), 0, a.stream,
                       static_cast<const TQ*>(a.qkv), static_cast<TQ*>(a.ctx), a.seq_len, a.heads, c2, nullptr,
                       nwords);
  return hipGetLastError();
}

template <int HD, int NW, int BN, int ST, bool CAUSAL, typename TQ>
static hipError_t launch_attn(const AttnArgs& a, float c2) {
  constexpr int BM = 32 * NW;
  const int nqb = (a.seq_len + BM - 1) / BM;
  const int64_t grid = (int64_t)nqb * a.heads * a.batch;
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  const int nwords = (int)mask_words(a.seq_len);
  if (a.key_bits)
    hipLaunchKernelGGL((attn_fwd_kernel<HD, NW, BN, ST, CAUSAL, true, TQ>), dim3((unsigned)grid), dim3(NW * 64), 0,
                       a.stream, static_cast<const TQ*>(a.qkv), static_cast<TQ*>(a.ctx), a.seq_len, a.heads,
                       a.head_dim, c2, nqb, a.key_bits, nwords);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<HD, NW, BN, ST, CAUSAL, false, TQ>), dim3((unsigned)grid), dim3(NW * 64), 0,
                       a.stream, static_cast<const TQ*>(a.qkv), static_cast<TQ*>(a.ctx), a.seq_len, a.heads,
                       a.head_dim, c2, nqb, nullptr, nwords);
  return hipGetLastError();
}

template <int HD, bool CAUSAL, typename TQ>
static hipError_t dispatch_waves(const AttnArgs& a, float c2) {
  // Waves per workgroup follow the sequence length: every K/V tile a
  // workgroup stages is shared by all of its waves, so long sequences take 8
  // (256 queries), short ones fewer so that no wave idles past S.  Wide heads
  // keep 4: the O accumulator already fills the register file.  Key blocks of
  // BN keys (one 1 KB DMA span per wave at least), ST stages deep.
  constexpr int BN = HD >= 256 ? 32 : 64;
  // 8-wave launches: at least one 1 KB span per wave per stage, and for narrow heads
  // 128-key blocks (half the barriers per key; +7-10 % at head_dim 32, measured)
  constexpr int BN8 = HD <= 32 ? 128 : BN;
  constexpr int ST = HD >= 128 ? 3 : 4;
  if constexpr (HD <= 64) {
    if (a.seq_len <= 32) return launch_attn<HD, 1, BN, ST, CAUSAL, TQ>(a, c2);
    if (a.seq_len <= 64) return launch_attn<HD, 2, BN, ST, CAUSAL, TQ>(a, c2);
  }
  if constexpr (HD <= 128) {
    if (a.seq_len > 128) return launch_attn<HD, 8, BN8, ST, CAUSAL, TQ>(a, c2);
  }
  return launch_attn<HD, 4, BN, ST, CAUSAL, TQ>(a, c2);
}

template <bool CAUSAL, typename TQ>
static hipError_t dispatch_hd(const AttnArgs& a, float c2) {
  const int hd = a.head_dim;
  // Wide heads over at most 128 keys: exact softmax, one workgroup per (sequence, head).
  if (a.seq_len <= 128 && hd == 256) return launch_attn_short<256, CAUSAL, TQ>(a, c2);
  if (a.seq_len <= 128 && hd == 128) return launch_attn_short<128, CAUSAL, TQ>(a, c2);
  if (hd <= 16) return dispatch_waves<16, CAUSAL, TQ>(a, c2);
  if (hd <= 32) return dispatch_waves<32, CAUSAL, TQ>(a, c2);
  if (hd <= 64) return dispatch_waves<64, CAUSAL, TQ>(a, c2);
  if (hd <= 128) return dispatch_waves<128, CAUSAL, TQ>(a, c2);
  return dispatch_waves<256, CAUSAL, TQ>(a, c2);
}

// One wave per 64-bit word: lane j reads the byte of key 64w + j (coalesced)
// and the ballot of "valid" is the word.
__global__ __launch_bounds__(256) void mask_bits_kernel(const uint8_t* __restrict__ mask, uint64_t* __restrict__ bits,
                                                        int64_t total_words, int S, int nw) {
  const int64_t word = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (word >= total_words) return;  // whole waves only
  const int lane = threadIdx.x & 63;
  const int64_t b = word / nw;
  const int key = (int)(word - b * nw) * 64 + lane;
  const bool valid = key < S && mask[b * S + key] != 0;
  const uint64_t v = __builtin_amdgcn_ballot_w64(valid);
  if (lane == 0) bits[word] = v;
}

hipError_t run_mask_bits(const uint8_t* mask, uint64_t* bits, int64_t batch, int seq_len, hipStream_t stream) {
  if (!mask || !bits || batch < 0 || seq_len < 0) return hipErrorInvalidValue;
  const int nw = (int)mask_words(seq_len);
  const int64_t total = batch * nw;
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + 3) / 4;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(mask_bits_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, mask, bits, total, seq_len, nw);
  return hipGetLastError();
}

hipError_t run_attn(const AttnArgs& a) {
  if (!a.qkv || !a.ctx || a.batch < 0 || a.seq_len < 0 || a.heads <= 0) return hipErrorInvalidValue;
  if (a.head_dim <= 0 || a.head_dim % 8 != 0 || a.head_dim > 256) return hipErrorInvalidValue;
  if (a.batch == 0 || a.seq_len == 0) return hipSuccess;
  const float c2 = a.scale * 1.4426950408889634f;  // scale * log2(e): softmax in the exp2 domain
  if (a.dtype == kBF16) return a.causal ? dispatch_hd<true, bf16>(a, c2) : dispatch_hd<false, bf16>(a, c2);
  if (a.dtype != kF16) return hipErrorInvalidValue;
  return a.causal ? dispatch_hd<true, f16>(a, c2) : dispatch_hd<false, f16>(a, c2);
}

}  // namespace cobra
