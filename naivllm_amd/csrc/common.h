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

// 16 bytes a kernel reads exactly once (K/V pages, projection weights,
// acceptance logits): a non-temporal load (the nt cache policy: no reuse
// expected, so the line is not kept), which streams faster than a default
// load that allocates in every cache level.  MI355X, graph-replayed: verify
// attention config 2 15.65 -> 14.8 us per call, config 4 329 -> 309 us; the
// Qwen3-0.6B round b1 1.114 -> 1.090 ms; stochastic acceptance 52.1 -> 50.9 us.
__device__ __forceinline__ u32x4 load16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// n / d for 0 <= n < 2^22 and d >= 1 through an fp32 reciprocal (relative
// error ~2^-22, so the truncated estimate is within one of the quotient) and
// one correction: a few instructions where the integer division sequence is
// ~25, on the attention kernels' paths to their first loads.
__device__ __forceinline__ int div_small(int n, int d) {
  int q = (int)((float)n * __builtin_amdgcn_rcpf((float)d));
  const int r = n - q * d;
  q += (r >= d) - (r < 0);
  return q;
}

// Raw 16-bit pattern of a bf16 value and back; bf16 is the upper half of an
// IEEE-754 binary32, so widening is a shift.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Two floats to packed bf16 (lo in the low half), round to nearest even: one
// v_cvt_pk_bf16_f32 on gfx950.  The same values as f32_to_bf16_bits below
// for every non-NaN input (a NaN comes out as a quiet NaN either way).
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){lo, hi}, bf16x2v));
}

// Round-to-nearest-even narrowing (a NaN stays a quiet NaN), the rounding
// torch and the reference's Triton `.to(bfloat16)` apply: gfx950's
// conversion instruction, one VALU operation.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) { return (uint16_t)pack_bf16x2(f, 0.f); }


// ---------------------------------------------------------------------------
// Wave reductions on the VALU: four DPP steps combine each 16-lane row
// (lane ^ 1, lane ^ 2, then the 8- and 16-lane mirrors, each pairing lanes
// that hold different partial results), then the four row results are read
// out with v_readlane and combined in the order row 0, 1, 2, 3.  No step goes
// through the LDS pipe, whose ds_bpermute round trip (~100+ cycles) would
// otherwise chain six times per reduction.  The result is uniform and the
// combination order is fixed, so floating-point sums are deterministic.
// ---------------------------------------------------------------------------
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within 16 lanes

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  return (uint64_t)dpp_u32<CTRL>((uint32_t)v) | ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32);
}
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}
__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int lane) {
  return (uint64_t)lane_u32((uint32_t)v, lane) | ((uint64_t)lane_u32((uint32_t)(v >> 32), lane) << 32);
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppMirror>(v));
  const float r0 = __uint_as_float(lane_u32(__float_as_uint(v), 0)), r1 = __uint_as_float(lane_u32(__float_as_uint(v), 16));
  const float r2 = __uint_as_float(lane_u32(__float_as_uint(v), 32)), r3 = __uint_as_float(lane_u32(__float_as_uint(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ double wave_sum_dpp(double v) {
  auto step = [](double x, double y) { return x + y; };
  uint64_t u = (uint64_t)__double_as_longlong(v);
  v = step(v, __longlong_as_double((long long)dpp_u64<kDppXor1>(u)));
  u = (uint64_t)__double_as_longlong(v);
  v = step(v, __longlong_as_double((long long)dpp_u64<kDppXor2>(u)));
  u = (uint64_t)__double_as_longlong(v);
  v = step(v, __longlong_as_double((long long)dpp_u64<kDppHalfMirror>(u)));
  u = (uint64_t)__double_as_longlong(v);
  v = step(v, __longlong_as_double((long long)dpp_u64<kDppMirror>(u)));
  u = (uint64_t)__double_as_longlong(v);
  const double r0 = __longlong_as_double((long long)lane_u64(u, 0)), r1 = __longlong_as_double((long long)lane_u64(u, 16));
  const double r2 = __longlong_as_double((long long)lane_u64(u, 32)), r3 = __longlong_as_double((long long)lane_u64(u, 48));
  return ((r0 + r1) + r2) + r3;
}

__device__ __forceinline__ float wave_sum_f32_dpp(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppHalfMirror>(v);
  v += dpp_f32<kDppMirror>(v);
  const float r0 = __uint_as_float(lane_u32(__float_as_uint(v), 0)), r1 = __uint_as_float(lane_u32(__float_as_uint(v), 16));
  const float r2 = __uint_as_float(lane_u32(__float_as_uint(v), 32)), r3 = __uint_as_float(lane_u32(__float_as_uint(v), 48));
  return ((r0 + r1) + r2) + r3;
}

// Maximum and sum over the 64 lanes of a wave (every lane active), uniform.
__device__ __forceinline__ float wave_max(float v) { return wave_max_dpp(v); }
__device__ __forceinline__ float wave_sum(float v) { return wave_sum_f32_dpp(v); }

__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t v) {
  auto mx = [](uint64_t x, uint64_t y) { return x > y ? x : y; };
  v = mx(v, dpp_u64<kDppXor1>(v));
  v = mx(v, dpp_u64<kDppXor2>(v));
  v = mx(v, dpp_u64<kDppHalfMirror>(v));
  v = mx(v, dpp_u64<kDppMirror>(v));
  return mx(mx(lane_u64(v, 0), lane_u64(v, 16)), mx(lane_u64(v, 32), lane_u64(v, 48)));
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

// Stores / loads with the cache policy of agent-scope (device-coherent)
// accesses (sc1: written through to, and read from, the device's point of
// coherence), through a buffer resource whose wave-uniform base is the
// caller's block: one instruction per 4 floats instead of two 64-bit
// atomics.  Nothing needs them single-copy atomic where readers load only
// after every writer's stores were acknowledged (the in-kernel merges).
constexpr int kCpolSc1 = 16;
// the non-temporal policy of a buffer load (as load16_stream's)
constexpr int kCpolNt = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
// Offsets: a per-lane byte offset plus a wave-uniform one.
__device__ __forceinline__ void store16_agent(__amdgpu_buffer_rsrc_t r, unsigned byte_off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)byte_off, 0, kCpolSc1);
}
__device__ __forceinline__ f32x4 load16_agent(__amdgpu_buffer_rsrc_t r, unsigned byte_off, unsigned uniform_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, (int)uniform_off, kCpolSc1));
}
__device__ __forceinline__ float2 load8_agent(__amdgpu_buffer_rsrc_t r, unsigned byte_off, unsigned uniform_off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)byte_off, (int)uniform_off, kCpolSc1);
  return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
}

// Workgroup barrier that orders LDS accesses only: unlike __syncthreads() it
// does not wait for the wave's outstanding global loads, so a load pipeline
// issued before it stays in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

static inline int nsv_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSV_OK : (int)e;
}
