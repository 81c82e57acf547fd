// Helpers shared by the fused attention-sublayer kernels (persistent and
// query-split variants): fragment conversions, stores, the fused plan's
// shape limits.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace cobra {

__device__ __forceinline__ void store4(f16* p, const float (&v)[4]) {
  f16x4 h;
#pragma unroll
  for (int i = 0; i < 4; ++i) h[i] = (f16)v[i];
  *reinterpret_cast<f16x4*>(p) = h;
}
__device__ __forceinline__ void store4(float* p, const float (&v)[4]) {
  f32x4 a;
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = v[i];
  *reinterpret_cast<f32x4*>(p) = a;
}

// A zero the optimiser cannot see through.  Offsetting the parameter
// pointers by it inside the persistent sequence loop keeps their loads in the
// loop (hoisting them would pin every LayerNorm and bias parameter in
// registers for the kernel's lifetime) while the pointers stay global.
__device__ __forceinline__ int opaque_zero() {
  int z = 0;
  asm volatile("" : "+s"(z));
  return z;
}

// Registers 8*half .. 8*half+7 of a 32x32 accumulator times `scale`, as fp16.
__device__ __forceinline__ f16x8 scaled_f16(const f32x16& acc, int half, float scale) {
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (f16)(acc[8 * half + e] * scale);
  return o;
}

// Registers 8*half .. 8*half+7 of a 32x32 accumulator, as fp16.
__device__ __forceinline__ f16x8 acc_f16(const f32x16& acc, int half) {
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (f16)acc[8 * half + e];
  return o;
}

// Adds the eight fp16 probabilities of `p` into two fp32 partial sums (v_dot2 against
// ones: half the instructions of fp32 adds).  The row sum is thereby taken over the
// rounded values that the P.V product consumes.
__device__ __forceinline__ void add_probs(const f16x8& p, float& a, float& b) {
  const f16x2 one2 = {(f16)1.0f, (f16)1.0f};
  a = __builtin_amdgcn_fdot2(f16x2{p[0], p[1]}, one2, a, false);
  b = __builtin_amdgcn_fdot2(f16x2{p[2], p[3]}, one2, b, false);
  a = __builtin_amdgcn_fdot2(f16x2{p[4], p[5]}, one2, a, false);
  b = __builtin_amdgcn_fdot2(f16x2{p[6], p[7]}, one2, b, false);
}

// Registers 8*half .. 8*half+7 of a 32x32 accumulator (+ per-register bias), as fp16.
__device__ __forceinline__ f16x8 half_to_f16(const f32x16& acc, int half, const float (&bias)[16]) {
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (f16)(acc[8 * half + e] + bias[8 * half + e]);
  return o;
}

// ---- token masks in the fused kernels (S <= 128) ----------------------------
// The validity of the (at most 128) keys of a sequence lives in two wave-uniform
// 64-bit words: lane j reads the mask bytes of keys j and 64 + j, and the two
// ballots are the words.  Keys past S count as padded.
struct KeyBytes {
  uint8_t lo, hi;
};
__device__ __forceinline__ KeyBytes load_key_bytes(const uint8_t* __restrict__ mrow, int S, int lane) {
  return {mrow[min(lane, S - 1)], mrow[min(64 + lane, S - 1)]};
}
// (Selects, not array indexing: a per-lane index into a private array makes the
// compiler move the array to LDS, and an LDS store behind in-flight LDS-DMA
// costs a wait for every transfer.)
struct KeyBits {
  uint64_t lo, hi;  // keys 0..63, 64..127
  // bits of keys 32t .. 32t+31 (t < 4)
  __device__ __forceinline__ uint32_t tile(int t) const { return (uint32_t)((t < 2 ? lo : hi) >> (32 * (t & 1))); }
  __device__ __forceinline__ bool valid(int key) const { return ((key < 64 ? lo : hi) >> (key & 63)) & 1; }
};
__device__ __forceinline__ KeyBits key_bits_of(KeyBytes kb, int S, int lane) {
  return {__builtin_amdgcn_ballot_w64(lane < S && kb.lo != 0), __builtin_amdgcn_ballot_w64(64 + lane < S && kb.hi != 0)};
}

// Padded keys of a 32-key score tile in the S^T = K Q^T layout (register r of
// lane (li, g) holds key 8(r/4) + 4g + r%4 of the tile) get -inf.
__device__ __forceinline__ void mask_key_tile(f32x16& s, uint32_t tile_bits, int g) {
  const uint32_t lw = tile_bits >> (4 * g);
#pragma unroll
  for (int r = 0; r < 16; ++r)
    if (!((lw >> (8 * (r >> 2) + (r & 3))) & 1)) s[r] = kNegInf;
}

// One step of the exact two-block softmax when keys may be masked: a query's
// running max starts at -inf and is set by the first block with a valid key
// for it; until then every probability is exp2(-inf) = 0.  Returns the offset
// the block's probabilities are taken against and the rescale of the
// running sum / output (0 while nothing was accumulated).
struct SoftmaxStep {
  float m_use, alpha;
};
__device__ __forceinline__ SoftmaxStep masked_softmax_step(float& m_run, float block_max_scaled) {
  const float m_new = fmaxf(m_run, block_max_scaled);
  const float m_use = m_new == kNegInf ? 0.f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
  m_run = m_new;
  return {m_use, alpha};
}

constexpr int kSmallMaxS = 128;
constexpr int kSmallWaves = kSmallMaxS / 32;  // one wave per 32-token tile; always launched in full
constexpr int kLdsBytes = 163840;  // gfx950: LDS per workgroup

template <typename TX>
struct XChunks;
template <>
struct XChunks<f16> {
  using c8 = f16x8;
  using c4 = f16x4;
};
template <>
struct XChunks<float> {
  using c8 = float __attribute__((ext_vector_type(8)));
  using c4 = f32x4;
};

// The value `v` of the partner lane (lane ^ 32), any 4-byte-multiple type, through
// The value of the partner lane (lane ^ 32), from one v_permlane32_swap per dword: of
// the swap's two results one is this lane's own value, the other the partner's (which
// is which depends on the half; equal bits either way).
template <typename V>
__device__ __forceinline__ V partner_value(const V& v) {
  constexpr int NDW = sizeof(V) / 4;
  static_assert(NDW * 4 == sizeof(V), "whole dwords");
  struct Dw {
    uint32_t u[NDW];
  };
  const Dw in = __builtin_bit_cast(Dw, v);
  Dw out;
#pragma unroll
  for (int d = 0; d < NDW; ++d) {
    const auto r = __builtin_amdgcn_permlane32_swap(in.u[d], in.u[d], false, false);
    out.u[d] = r[0] == in.u[d] ? r[1] : r[0];
  }
  return __builtin_bit_cast(V, out);
}

// Lane-pair exchange of two values in one v_permlane32_swap per dword: the swap trades
// the upper 32 lanes of its first operand for the lower 32 lanes of its second, so
// afterwards lanes l < 32 hold (a, a of lane l + 32) and lanes l >= 32 hold
// (b of lane l - 32, b).  With a, b the two halves of what a lane pair must regroup
// (lane l keeps the pieces of half 0, lane l + 32 those of half 1), no selects are needed.
template <typename V>
__device__ __forceinline__ void swap_halves(V& a, V& b) {
  constexpr int NDW = sizeof(V) / 4;
  static_assert(NDW * 4 == sizeof(V), "whole dwords");
  struct Dw {
    uint32_t u[NDW];
  };
  Dw x = __builtin_bit_cast(Dw, a), y = __builtin_bit_cast(Dw, b);
#pragma unroll
  for (int d = 0; d < NDW; ++d) {
    const auto r = __builtin_amdgcn_permlane32_swap(x.u[d], y.u[d], false, false);
    x.u[d] = r[0];
    y.u[d] = r[1];
  }
  a = __builtin_bit_cast(V, x);
  b = __builtin_bit_cast(V, y);
}

// Query-split variant of the fused kernel (layer_split.hip): fp16
// activations at d_model 64 / 128 (head_dim 32 / 64, and 8 or 128 at d_model 128),
// while batch * ceil(S/32) workgroups take at most two rounds of the chip.
bool layer_split_ok(int64_t seq_len, int64_t d_model, int64_t heads);
bool layer_split_pays(int64_t batch, int64_t seq_len, int64_t d_model, int x_dtype);
hipError_t run_layer_split(const SmallLayerArgs& a);

}  // namespace cobra
