// Shared device helpers for the CDNA4 (gfx950) kernels of the attention sublayer.
//
// Matrix-core conventions used by every kernel (v_mfma_f32_32x32x16_f16, wave64):
//   A operand (32 x 16, M x K): lane l holds row (l % 32), k = 8*(l / 32) + e, e = 0..7
//   B operand (16 x 32, K x N): lane l holds col (l % 32), k = 8*(l / 32) + e
//   C/D (32 x 32, fp32, 16 regs): lane l, reg r holds
//        row = 8*(r / 4) + 4*(l / 32) + (r % 4),  col = l % 32
// Only the pairing of A and B along k matters for a product, so a kernel may
// feed any permutation of k as long as both operands use the same one; the
// attention kernel relies on that to use softmax output registers directly as
// an operand.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cobra {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// bfloat16 (8-bit mantissa, fp32's exponent range): conversions from fp32 round to
// nearest even (v_cvt_pk_bf16_f32), to fp32 are exact.
typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// dtype codes of the C ABI (include/cobra_amd.h)
enum : int { kF16 = 0, kF32 = 1, kBF16 = 2 };

// 16-bit MFMA operand types: T is f16 or bf16; V8 / V4 / V2 its 8 / 4 / 2-element vectors.
template <typename T>
struct Op16;
template <>
struct Op16<f16> {
  typedef f16x8 V8;
  typedef f16x4 V4;
  typedef f16x2 V2;
};
template <>
struct Op16<bf16> {
  typedef bf16x8 V8;
  typedef bf16x4 V4;
  typedef bf16x2 V2;
};

constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ f32x16 mfma32x32x16(const f16x8& a, const f16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// acc + a.x * b.x + a.y * b.y with fp32 accumulation (v_dot2_f32_f16 / v_dot2_f32_bf16).
__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float acc) { return __builtin_amdgcn_fdot2(a, b, acc, false); }
__device__ __forceinline__ float dot2(bf16x2 a, bf16x2 b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(a, b, acc, false);
}

// a - b on both fp16 halves as one v_pk_add_f16 (with the second operand
// negated): the compiler lowers fp16 vector arithmetic to one instruction per
// half on this target.
__device__ __forceinline__ f16x2 pk_sub_f16(f16x2 a, f16x2 b) {
  f16x2 r;
  asm("v_pk_add_f16 %0, %1, %2 neg_lo:[0,1] neg_hi:[0,1]" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// (x - hi) - lo elementwise, in packed fp16 (two roundings, each relative to the result).
__device__ __forceinline__ f16x8 sub2_f16(const f16x8& x, _Float16 hi, _Float16 lo) {
  struct Pairs {
    f16x2 p[4];
  };
  const f16x2 h2 = {hi, hi}, l2 = {lo, lo};
  Pairs q = __builtin_bit_cast(Pairs, x);
#pragma unroll
  for (int i = 0; i < 4; ++i) q.p[i] = pk_sub_f16(pk_sub_f16(q.p[i], h2), l2);
  return __builtin_bit_cast(f16x8, q);
}

__device__ __forceinline__ f16x8 zero8() {
  f16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (f16)0.0f;
  return z;
}
// Eight zeros of a 16-bit operand type.
template <typename T>
__device__ __forceinline__ typename Op16<T>::V8 zero8_of() {
  typename Op16<T>::V8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (T)0.0f;
  return z;
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// Cross-lane exchanges on the vector ALU (no LDS round trip, unlike the
// ds_bpermute behind __shfl_xor).  v_permlane32_swap / v_permlane16_swap
// exchange 32- / 16-lane halves of two registers; passing the same register
// twice yields, in the two results, the value of this lane and of lane ^ 32
// (^ 16), in an order that depends on the half -- so the sum or max below is
// the same bitwise in both lanes of a pair.
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// One value common to both lanes of a pair (l, l ^ 32): v of one of the two
// lanes.  The first result of the swap holds the same lane's value in both
// halves (which lane depends only on the operand order), so the pair agrees.
__device__ __forceinline__ f16 pair_pilot(f16 v) {
  const uint32_t u = __builtin_bit_cast(uint16_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(f16, (uint16_t)r[0]);
}
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v of another lane of the same 16-lane row, chosen by a DPP control word.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of W lanes (W a power of two <= 64); every lane of
// the group receives the same group total.  All 64 lanes must execute it.
// Butterfly on DPP lane swizzles: lane ^ 1 and lane ^ 2 (quad_perm), the
// other quad of an 8-lane group (row_half_mirror), the other half of a 16-lane
// row (row_mirror), then lane ^ 16 and lane ^ 32.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
  if constexpr (W >= 2) v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (W >= 4) v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v += dpp_f32<0x141>(v);  // row_half_mirror
  if constexpr (W >= 16) v += dpp_f32<0x140>(v); // row_mirror
  if constexpr (W >= 32) v = sum_xor16(v);
  if constexpr (W >= 64) v = sum_xor32(v);
  return v;
}

// 8 consecutive elements <-> fp32 registers.
__device__ __forceinline__ void load8(const f16* p, float (&v)[8]) {
  const f16x8 h = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
}
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = a[i];
    v[i + 4] = b[i];
  }
}
__device__ __forceinline__ void load8(const bf16* p, float (&v)[8]) {
  const bf16x8 h = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
}
// Eight consecutive elements of a row as loaded (fp16: one 16-byte load; fp32:
// two), converted to fp32 only when used, so that loads in flight hold half the
// registers for fp16 rows.
template <typename TX>
struct RowChunk;
template <>
struct RowChunk<f16> {
  f16x8 v;
};
template <>
struct RowChunk<float> {
  f32x4 lo, hi;
};
template <>
struct RowChunk<bf16> {
  bf16x8 v;
};
__device__ __forceinline__ RowChunk<f16> load_chunk(const f16* p) { return {*reinterpret_cast<const f16x8*>(p)}; }
__device__ __forceinline__ RowChunk<float> load_chunk(const float* p) {
  return {*reinterpret_cast<const f32x4*>(p), *reinterpret_cast<const f32x4*>(p + 4)};
}
__device__ __forceinline__ RowChunk<bf16> load_chunk(const bf16* p) { return {*reinterpret_cast<const bf16x8*>(p)}; }
__device__ __forceinline__ void to_float8(const RowChunk<bf16>& c, float (&v)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (float)c.v[e];
}
__device__ __forceinline__ void to_float8(const RowChunk<f16>& c, float (&v)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (float)c.v[e];
}
__device__ __forceinline__ void to_float8(const RowChunk<float>& c, float (&v)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = c.lo[e];
    v[4 + e] = c.hi[e];
  }
}

__device__ __forceinline__ void store8(f16* p, const float (&v)[8]) {
  f16x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (f16)v[i];
  *reinterpret_cast<f16x8*>(p) = h;
}
__device__ __forceinline__ void store8(bf16* p, const float (&v)[8]) {
  bf16x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (bf16)v[i];
  *reinterpret_cast<bf16x8*>(p) = h;
}
__device__ __forceinline__ void store8(float* p, const float (&v)[8]) {
  f32x4 a, b;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = v[i];
    b[i] = v[i + 4];
  }
  *reinterpret_cast<f32x4*>(p) = a;
  *reinterpret_cast<f32x4*>(p + 4) = b;
}

// Exact (erf) GELU, F.gelu(approximate="none"), in the reference epilogue's
// operation order: v * 0.5 * (1 + erf(v / sqrt(2))) (TTB:326-328).
__device__ __forceinline__ float gelu_erf(float v) { return v * 0.5f * (1.0f + erff(v * 0.7071067811865476f)); }

// The same GELU without branches, for epilogues where a handful of values per lane
// sit on the critical path: erf from Abramowitz & Stegun 7.1.26,
//   erf(z) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2),  t = 1 / (1 + p z),
// |error| <= 1.5e-7 for z >= 0 (one reciprocal, one exp2, six fma).  1 + erf(v / sqrt 2) is
// formed as 2 - q (v >= 0) or q (v < 0) with q = 1 - erf(|v| / sqrt 2), so the negative
// tail keeps its small values instead of cancelling against 1.
__device__ __forceinline__ float gelu_erf_fast(float v) {
  const float z = fabsf(v) * 0.7071067811865476f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));
  float poly = fmaf(1.061405429f, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  const float q = poly * t * __builtin_amdgcn_exp2f(v * v * -0.7213475204444817f);  // exp(-v^2 / 2)
  return v * 0.5f * (v >= 0.f ? 2.0f - q : q);
}

// Workgroup-id remap so that consecutive logical tiles land on the same XCD
// (the hardware deals workgroups round-robin over 8 XCDs, each with its own
// L2).  A bijection on [0, n) for any n.
__device__ __forceinline__ int xcd_remap(int id, int n) {
  constexpr int kXcd = 8;
  if (n < kXcd) return id;
  const int per = (n + kXcd - 1) / kXcd;  // ids per XCD, rounded up
  int tall = n % kXcd;                    // XCDs that get `per` ids
  if (tall == 0) tall = kXcd;
  const int xcd = id % kXcd, local = id / kXcd;
  return xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
}

}  // namespace cobra
