// Shared device helpers for the gfx950 kernels of libnaivspec.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/naivspec.h"

typedef __bf16 bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define NSV_WAVE 64

// Raw 16-bit pattern of a bf16 value and back; bf16 is the upper half of an
// IEEE-754 binary32, so widening is a shift.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even narrowing (NaN kept quiet), the rounding torch and
// the reference's Triton `.to(bfloat16)` apply.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, NSV_WAVE));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, NSV_WAVE);
  return v;
}

// Per-head q/k RMSNorm and NeoX rotation of one rotation pair (x1, x2) =
// (row[l], row[l + D/2]), with floating-point contraction off: every caller
// evaluates the same IEEE operations (no fused multiply-add chosen per call
// site), so a row comes out bit-identical wherever it is computed.
__device__ __forceinline__ float head_sq(float x1, float x2) {
#pragma clang fp contract(off)
  return x1 * x1 + x2 * x2;
}
__device__ __forceinline__ float head_inv_rms(float sum_sq, int D, float eps) {
#pragma clang fp contract(off)
  return rsqrtf(sum_sq / (float)D + eps);
}
// The normalised pair is rounded to bf16 (the reference's q_norm / k_norm
// output) before the rotation by the row's (cos, sin).
__device__ __forceinline__ void head_norm_rope(float x1, float x2, float inv, float w1, float w2, float c, float s,
                                               uint16_t& o1, uint16_t& o2) {
#pragma clang fp contract(off)
  const float y1 = bf16_bits_to_f32(f32_to_bf16_bits(x1 * inv * w1));
  const float y2 = bf16_bits_to_f32(f32_to_bf16_bits(x2 * inv * w2));
  o1 = f32_to_bf16_bits(y1 * c - y2 * s);
  o2 = f32_to_bf16_bits(y1 * s + y2 * c);
}

static inline int nsv_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSV_OK : (int)e;
}
