// Flash-style multi-head attention over a packed qkv buffer, causal or not.
//
// Replaces the reference's _attn_kernel / _attn_cfgs / _tl_attn
// (torch_transformer_benchmark.py:572-649, 788-854), which is causal-only, and
// the SDPA call the reference uses for non-causal attention (TTB:1240-1253).
// Semantics per query row i (TTB:98-113): s_j = (q_i . k_j) * scale, masked
// keys (j > i under causality, j >= S) are -inf, p = softmax(s) in fp32,
// ctx_i = sum_j p_j v_j.  The [S, S] score matrix is never formed: keys are
// visited in blocks with an online (running max / running sum) softmax in the
// exp2 domain, normalised once at the end.
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
//     (no padding, conflict-free operand reads), double-buffered: the next key
//     block is prefetched into registers during the matrix work and stored to
//     the other buffer, one barrier per block;
//   * lazy rescale: a query's running max only moves (rescaling O and the sum)
//     when a block raises it by more than 2^8 -- the probabilities stay below
//     256, well inside fp16 -- and the whole wave skips the rescale when no
//     lane needs it.
#include "common.hpp"
#include "kernels.hpp"

namespace cobra {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f16x4 lds_read_tr16(const f16* p) {
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  return __builtin_bit_cast(f16x4, r);
}

// Chunk swizzle of a [rows][HD] fp16 tile: 16-byte chunk c of row r lives at
// chunk c ^ swz(r).  Any 16 consecutive rows reading one chunk column hit 16
// distinct 4-bank groups.
template <int HD>
__device__ __forceinline__ int swz(int row) {
  constexpr int kRowsPer256B = HD >= 128 ? 1 : 128 / HD;
  constexpr int kMask = (HD / 8 < 16 ? HD / 8 : 16) - 1;
  return (row / kRowsPer256B) & kMask;
}

constexpr float kLazyRescale = 8.0f;  // log2 units

}  // namespace

template <int HD, int NW, int BN, bool CAUSAL>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(const f16* __restrict__ qkv, f16* __restrict__ ctx,
                                                           int S, int H, int hd, float c2, int nqb) {
  constexpr int BM = 32 * NW;          // queries per workgroup
  constexpr int KS = HD / 16;          // k-steps of the QK^T product
  constexpr int ND = (HD + 31) / 32;   // 32-row blocks of d in O^T
  constexpr int NT = NW * 64;
  constexpr int CPR = HD / 8;          // 16-byte chunks per key row
  constexpr int CH = BN * CPR;         // chunks per tile
  constexpr int IT = (CH + NT - 1) / NT;
  static_assert(HD % 16 == 0 && BN % 32 == 0, "tile geometry");

  __shared__ __attribute__((aligned(16))) f16 Ks[2][BN * HD];
  __shared__ __attribute__((aligned(16))) f16 Vs[2][BN * HD];

  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int qb = id % nqb;
  const int bh = id / nqb;
  const int h = bh % H;
  const int64_t b = bh / H;
  const int D = H * hd;
  const int64_t ld = 3 * (int64_t)D;
  const f16* qbase = qkv + b * S * ld + h * hd;
  const f16* kbase = qbase + D;
  const f16* vbase = qbase + 2 * D;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, li = lane & 31;
  const int q0w = qb * BM + w * 32;  // this wave's first query
  const int qi = q0w + li;           // this lane's query

  // Q^T fragments: B operand of S^T = K . Q^T (k = d).
  f16x8 qf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const int d0 = kk * 16 + g * 8;
    qf[kk] = (qi < S && d0 < hd) ? *reinterpret_cast<const f16x8*>(qbase + qi * ld + d0) : zero8();
  }

  f16x8 rk[IT], rv[IT];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * NT;
      const int key = kb + c / CPR;
      const int d0 = (c % CPR) * 8;
      const bool ok = (CH % NT == 0 || c < CH) && key < S && d0 < hd;
      rk[i] = ok ? *reinterpret_cast<const f16x8*>(kbase + key * ld + d0) : zero8();
      rv[i] = ok ? *reinterpret_cast<const f16x8*>(vbase + key * ld + d0) : zero8();
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * NT;
      if (CH % NT == 0 || c < CH) {
        const int row = c / CPR;
        const int off = row * HD + (((c % CPR) ^ swz<HD>(row)) * 8);
        *reinterpret_cast<f16x8*>(&Ks[buf][off]) = rk[i];
        *reinterpret_cast<f16x8*>(&Vs[buf][off]) = rv[i];
      }
    }
  };

  f32x16 o[ND];
#pragma unroll
  for (int j = 0; j < ND; ++j) o[j] = zero16();
  float m_run = 0.f;  // running max in the scaled (log2) domain, set by block 0
  float l_run = 0.f;  // this lane's share of the running sum

  // Per-lane V^T read geometry (see the header): row within a 16-key step,
  // column within a 32-wide d tile.
  const int vr = 4 * g + ((lane & 15) >> 2);
  const int vc = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  const int kend = CAUSAL ? min(S, (qb + 1) * BM) : S;
  const int nblk = (kend + BN - 1) / BN;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int n = 0; n < nblk; ++n) {
    const int kb = n * BN;
    const int cur = n & 1;
    const bool more = n + 1 < nblk;
    if (more) gload(kb + BN);
    const f16* Kc = Ks[cur];
    const f16* Vc = Vs[cur];

    f32x16 s[BN / 32];
#pragma unroll
    for (int t = 0; t < BN / 32; ++t) {
      s[t] = zero16();
      const int row = t * 32 + li;
      const f16* krow = Kc + row * HD;
      const int sw = swz<HD>(row);
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(krow + (((2 * kk + g) ^ sw) * 8));
        s[t] = mfma32x32x16(a, qf[kk], s[t]);
      }
    }

    // Masks only where a block reaches past S or, causally, past this wave's first query.
    if (kb + BN > S || (CAUSAL && kb + BN > q0w + 1)) {
#pragma unroll
      for (int t = 0; t < BN / 32; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb + t * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= S || (CAUSAL && key > qi)) s[t][r] = kNegInf;
        }
    }
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < BN / 32; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mc = mx * c2;
    if (n == 0) {
      m_run = mc;  // block 0 holds key 0, valid for every query: finite
    } else if (__builtin_amdgcn_ballot_w64(mc > m_run + kLazyRescale)) {
      const float m_new = fmaxf(m_run, mc);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int j = 0; j < ND; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[j][r] *= alpha;
      m_run = m_new;
    }

    f16x8 pf[BN / 16];
#pragma unroll
    for (int t = 0; t < BN / 32; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(s[t][r], c2, -m_run));
        l_run += p;
        pf[t * 2 + (r >> 3)][r & 7] = (f16)p;
      }

#pragma unroll
    for (int ks = 0; ks < BN / 16; ++ks)
#pragma unroll
      for (int j = 0; j < ND; ++j) {
        f16x4 lo, hi;
        if (HD >= 32 || vc < HD) {
          const int c = j * 32 + vc;
          const int r0 = ks * 16 + vr, r1 = r0 + 8;
          lo = lds_read_tr16(Vc + r0 * HD + (((c >> 3) ^ swz<HD>(r0)) * 8) + (c & 7));
          hi = lds_read_tr16(Vc + r1 * HD + (((c >> 3) ^ swz<HD>(r1)) * 8) + (c & 7));
        } else {
          lo = hi = f16x4{(f16)0.0f, (f16)0.0f, (f16)0.0f, (f16)0.0f};  // d beyond a 16-wide head
        }
        const f16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[j] = mfma32x32x16(a, pf[ks], o[j]);
      }

    if (more) sstore(cur ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (qi < S) {
    f16* out = ctx + (b * S + qi) * (int64_t)D + h * hd;
#pragma unroll
    for (int j = 0; j < ND; ++j)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = j * 32 + 8 * q4 + 4 * g;
        if (d < hd) {
          f16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (f16)(o[j][q4 * 4 + e] * inv);
          *reinterpret_cast<f16x4*>(out + d) = v;
        }
      }
  }
}

template <int HD, int NW, int BN, bool CAUSAL>
static hipError_t launch_attn(const AttnArgs& a, float c2) {
  constexpr int BM = 32 * NW;
  const int nqb = (a.seq_len + BM - 1) / BM;
  const int64_t grid = (int64_t)nqb * a.heads * a.batch;
  if (grid > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_fwd_kernel<HD, NW, BN, CAUSAL>), dim3((unsigned)grid), dim3(NW * 64), 0, a.stream,
                     static_cast<const f16*>(a.qkv), static_cast<f16*>(a.ctx), a.seq_len, a.heads, a.head_dim, c2,
                     nqb);
  return hipGetLastError();
}

template <int HD, bool CAUSAL>
static hipError_t dispatch_waves(const AttnArgs& a, float c2) {
  // Fewer waves per workgroup for short sequences, except at wide heads, where
  // the per-thread share of the K/V prefetch would no longer fit in registers.
  constexpr int BN = HD >= 256 ? 32 : 64;
  if constexpr (HD <= 64) {
    if (a.seq_len <= 32) return launch_attn<HD, 1, BN, CAUSAL>(a, c2);
    if (a.seq_len <= 64) return launch_attn<HD, 2, BN, CAUSAL>(a, c2);
  }
  return launch_attn<HD, 4, BN, CAUSAL>(a, c2);
}

template <bool CAUSAL>
static hipError_t dispatch_hd(const AttnArgs& a, float c2) {
  const int hd = a.head_dim;
  if (hd <= 16) return dispatch_waves<16, CAUSAL>(a, c2);
  if (hd <= 32) return dispatch_waves<32, CAUSAL>(a, c2);
  if (hd <= 64) return dispatch_waves<64, CAUSAL>(a, c2);
  if (hd <= 128) return dispatch_waves<128, CAUSAL>(a, c2);
  return dispatch_waves<256, CAUSAL>(a, c2);
}

hipError_t run_attn(const AttnArgs& a) {
  if (!a.qkv || !a.ctx || a.batch < 0 || a.seq_len < 0 || a.heads <= 0) return hipErrorInvalidValue;
  if (a.head_dim <= 0 || a.head_dim % 8 != 0 || a.head_dim > 256) return hipErrorInvalidValue;
  if (a.batch == 0 || a.seq_len == 0) return hipSuccess;
  const float c2 = a.scale * 1.4426950408889634f;  // scale * log2(e): softmax in the exp2 domain
  return a.causal ? dispatch_hd<true>(a, c2) : dispatch_hd<false>(a, c2);
}

}  // namespace cobra
