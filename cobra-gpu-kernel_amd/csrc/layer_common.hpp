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

// Registers 8*half .. 8*half+7 of a 32x32 accumulator (+ per-register bias), as fp16.
__device__ __forceinline__ f16x8 half_to_f16(const f32x16& acc, int half, const float (&bias)[16]) {
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (f16)(acc[8 * half + e] + bias[8 * half + e]);
  return o;
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

// Query-split variant of the fused kernel (layer_split.hip): fp16
// activations at d_model 64 / 128, while batch * ceil(S/32) workgroups take at
// most two rounds of the chip.
bool layer_split_pays(int64_t batch, int64_t seq_len, int64_t d_model, int x_dtype);
hipError_t run_layer_split(const SmallLayerArgs& a, float c2);

}  // namespace cobra
