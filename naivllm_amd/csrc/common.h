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

static inline int nsv_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSV_OK : (int)e;
}
