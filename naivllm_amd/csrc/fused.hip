// Fused elementwise stages of the Qwen3 verify forward for gfx950 (bf16).
//
// The reference composes these from separate torch ops (each a kernel
// launch and an HBM round trip of the activations):
//   * residual add + RMSNorm: layers/layernorm.py:18-35;
//   * per-head q/k RMSNorm, NeoX rotary embedding and the paged KV store:
//     models/qwen3.py:100-119, layers/rotary_embedding.py:4-86 and
//     layers/attention.py:9-112 (store_kvcache) -- the pre-attention
//     epilogue, one kernel here;
//   * SiLU(gate) * up: layers/activation.py:17-19.
// Arithmetic is fp32 inside each kernel with one bf16 rounding per output.

#include "common.h"

namespace {

__device__ __forceinline__ float bf(uint16_t b) { return bf16_bits_to_f32(b); }

// ---------------------------------------------------------------------------
// out = rmsnorm(r) * w, r = x + residual (residual may be null: r = x);
// r is written to residual_out when given.  One workgroup per row.
// ---------------------------------------------------------------------------
constexpr int kNormThreads = 256;

template <int J>  // elements per thread: E <= 256 J
__global__ __launch_bounds__(kNormThreads) void rms_norm_residual_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ residual, uint16_t* __restrict__ residual_out,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int E, float eps) {
  __shared__ float red[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * E;
  const uint16_t* rr = residual ? residual + row * E : xr;
  float ss = 0.f;
  // thread t handles elements t, t + 256, ... (E <= J * 256), kept in
  // registers; every load (the norm weight's included) is issued before the
  // first is used, elements past E reading element E - 1 (one round trip)
  uint16_t xv[J], rv[J], wv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = min((int)threadIdx.x + j * kNormThreads, E - 1);
    xv[j] = xr[i];
    rv[j] = rr[i];
    wv[j] = w[i];
  }
  // (used here, so that no load is moved into the residual branch below)
#pragma unroll
  for (int j = 0; j < J; ++j) __asm__ volatile("" ::"v"((uint32_t)rv[j]));
  float v[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = threadIdx.x + j * kNormThreads;
    float r = bf(xv[j]);
    if (residual) r = bf16_bits_to_f32(f32_to_bf16_bits(r + bf(rv[j])));  // the residual stream is bf16
    v[j] = i < E ? r : 0.f;
    ss += v[j] * v[j];
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
  const float inv = rsqrtf(tot / (float)E + eps);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = threadIdx.x + j * kNormThreads;
    if (i < E) {
      if (residual_out) residual_out[row * E + i] = f32_to_bf16_bits(v[j]);
      out[row * E + i] = f32_to_bf16_bits(v[j] * inv * bf(wv[j]));
    }
  }
}

// ---------------------------------------------------------------------------
// Forward prologue: r = embed[ids[t]] (the residual stream's first value,
// written to residual_out), out = rmsnorm(r) * w (layer 0's input norm), and
// the rotary table row of the row's position (position < 0 takes row 0) into
// rope_out [T, D] for every layer's epilogue.  An id outside [0, V) reads
// row 0, as the reference's lookup does on one GPU (the id times its in-range
// mask, layers/embedding_head.py:49-55).  One workgroup per row.
// ---------------------------------------------------------------------------
template <int J>  // elements per thread: E <= 256 J
__global__ __launch_bounds__(kNormThreads) void embed_norm_kernel(
    const int64_t* __restrict__ ids, const uint16_t* __restrict__ embed, int64_t V, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ residual_out, uint16_t* __restrict__ out, int E, float eps,
    const int64_t* __restrict__ positions, const float* __restrict__ cos_sin, int max_pos, int D,
    float* __restrict__ rope_out) {
  __shared__ float red[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  // first round trip: the id, the position and the norm weight (elements past
  // E read element E - 1); then the embedding row and the rotary row
  const int64_t id = ids[row];
  const int64_t pos_raw = rope_out ? positions[row] : 0;
  uint16_t wv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) wv[j] = w[min((int)threadIdx.x + j * kNormThreads, E - 1)];
  const bool valid = id >= 0 && id < V;
  const uint16_t* xr = embed + (valid ? id : 0) * E;
  uint16_t xv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) xv[j] = xr[min((int)threadIdx.x + j * kNormThreads, E - 1)];
  if (rope_out) {
    const int64_t pos = pos_raw < 0 ? 0 : (pos_raw >= max_pos ? max_pos - 1 : pos_raw);
    for (int i = threadIdx.x; i < D; i += kNormThreads) rope_out[row * D + i] = cos_sin[pos * D + i];
  }
  float ss = 0.f;
  float v[J];  // thread t holds elements t, t + 256, ...
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = threadIdx.x + j * kNormThreads;
    v[j] = i < E ? bf(xv[j]) : 0.f;
    ss += v[j] * v[j];
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
  const float inv = rsqrtf(tot / (float)E + eps);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = threadIdx.x + j * kNormThreads;
    if (i < E) {
      residual_out[row * E + i] = f32_to_bf16_bits(v[j]);
      out[row * E + i] = f32_to_bf16_bits(v[j] * inv * bf(wv[j]));
    }
  }
}

// ---------------------------------------------------------------------------
// Pre-attention epilogue.  qkv [T, (H + 2*Hkv) * D]: one wave per (row,
// head); lane l holds elements l and l + D/2 (exactly the NeoX rotation
// pair), D/2 <= 64.  q heads: RMSNorm * q_w, rotate, write q_out [T, H, D].
// k heads: RMSNorm * k_w, rotate, store at the row's slot.  v heads: store.
// Rows with slot < 0 store nothing; rows with position < 0 use position 0.
// With positions == NULL the rotary table holds one row per step row
// ([T, D], gathered at the rows' positions by the caller).
// ---------------------------------------------------------------------------
struct EpilogueArgs {
  const uint16_t* qkv;
  const uint16_t* q_w;
  const uint16_t* k_w;
  const float* cos_sin;  // [max_pos, D]: cos in [0, D/2), sin in [D/2, D); [T, D] by row without positions
  const int64_t* positions;
  const int64_t* slots;
  uint16_t* q_out;
  uint16_t* k_cache;  // [num_blocks * block_size, Hkv, D]
  uint16_t* v_cache;
  int T, H, Hkv, D, max_pos;
  float eps;
};

// Every load of a wave is issued at its start, in one round trip: the row's
// q/k/v head, its slot, the norm weight and (per-row table, POS false) the
// rotary row; with positions (POS true) the rotary row waits for the
// position.  Loads are unconditional (lanes past D/2 and waves past the last
// head read clamped elements and leave): a load under a branch is waited for
// on the spot.
template <bool POS>
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(EpilogueArgs a) {
  __asm__ volatile("" ::"s"(a.qkv), "s"(a.q_w), "s"(a.k_w), "s"(a.cos_sin), "s"(a.positions), "s"(a.slots),
                   "s"(a.q_out), "s"(a.k_cache), "s"(a.v_cache), "s"(a.T), "s"(a.H), "s"(a.Hkv), "s"(a.D),
                   "s"(a.max_pos), "s"(a.eps));
  const int heads = a.H + 2 * a.Hkv;
  const int wave_raw = (blockIdx.x * 256 + threadIdx.x) >> 6;  // 256 threads: the launch's block size
  const int wave = __builtin_amdgcn_readfirstlane(min(wave_raw, a.T * heads - 1));
  const int lane = threadIdx.x & 63;
  const int row = wave / heads, head = wave - row * heads;
  const int half = a.D >> 1;
  const bool on = lane < half;
  const int l = on ? lane : half - 1;
  const bool is_q = head < a.H, is_v = head >= a.H + a.Hkv;
  const uint16_t* src = a.qkv + ((int64_t)row * heads + head) * a.D;
  const uint16_t* w = is_q ? a.q_w : a.k_w;
  const uint16_t s1 = src[l], s2 = src[l + half];
  const int64_t slot = a.slots[row];
  const uint16_t w1 = w[l], w2 = w[l + half];
  int64_t pos = row;
  if constexpr (POS) {
    pos = a.positions[row];
    pos = pos < 0 ? 0 : (pos >= a.max_pos ? a.max_pos - 1 : pos);
  }
  const float c = a.cos_sin[pos * a.D + l], sn = a.cos_sin[pos * a.D + half + l];
  // (used here, so that no load is moved behind the branches below, which
  // only some heads take)
  __asm__ volatile("" ::"v"(s1), "v"(s2), "v"(w1), "v"(w2), "v"(c), "v"(sn));
  if (wave_raw >= a.T * heads) return;
  if (is_v) {  // v head: store as is
    if (on && slot >= 0) {
      uint16_t* dst = a.v_cache + (slot * a.Hkv + (head - a.H - a.Hkv)) * a.D;
      dst[lane] = s1;
      dst[lane + half] = s2;
    }
    return;
  }
  const float x1 = on ? bf(s1) : 0.f, x2 = on ? bf(s2) : 0.f;
  const float inv = head_inv_rms(wave_sum(head_sq(x1, x2)), a.D, a.eps);
  if (on) {
    uint16_t o1, o2;
    head_norm_rope(x1, x2, inv, bf(w1), bf(w2), c, sn, o1, o2);
    if (is_q) {
      uint16_t* dst = a.q_out + ((int64_t)row * a.H + head) * a.D;
      dst[lane] = o1;
      dst[lane + half] = o2;
    } else if (slot >= 0) {
      uint16_t* dst = a.k_cache + (slot * a.Hkv + (head - a.H)) * a.D;
      dst[lane] = o1;
      dst[lane + half] = o2;
    }
  }
}

// ---------------------------------------------------------------------------
// out[t, i] = silu(gu[t, i]) * gu[t, I + i]
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                       int64_t T, int I) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= T * I) return;
  const int64_t t = idx / I;
  const int i = (int)(idx - t * I);
  const float g = bf(gu[t * 2 * I + i]);
  const float u = bf(gu[t * 2 * I + I + i]);
  out[idx] = f32_to_bf16_bits(g / (1.f + __expf(-g)) * u);
}

}  // namespace

extern "C" {

int nsv_rms_norm(const void* x, const void* residual, void* residual_out, const void* weight, void* out, int T,
                 int E, float eps, void* stream) {
  if (T < 0 || E <= 0 || E > 16 * kNormThreads) return NSV_ERR_ARG;
  if (T == 0) return NSV_OK;
  if (!x || !weight || !out) return NSV_ERR_ARG;
  const int J = (E + kNormThreads - 1) / kNormThreads;
#define NSV_NORM(JJ)                                                                                              \
  hipLaunchKernelGGL(rms_norm_residual_kernel<JJ>, dim3(T), dim3(kNormThreads), 0, (hipStream_t)stream,          \
                     (const uint16_t*)x, (const uint16_t*)residual, (uint16_t*)residual_out,                     \
                     (const uint16_t*)weight, (uint16_t*)out, E, eps)
  if (J <= 4) NSV_NORM(4);
  else if (J <= 8) NSV_NORM(8);
  else NSV_NORM(16);
#undef NSV_NORM
  return nsv_launch_status();
}

int nsv_embed_rms_norm(const int64_t* ids, const void* embed, int64_t vocab, const void* weight, float eps,
                       void* residual_out, void* out, int T, int E, const int64_t* positions, const float* cos_sin,
                       int max_pos, int D, float* rope_out, void* stream) {
  if (T < 0 || E <= 0 || E > 16 * kNormThreads || vocab <= 0) return NSV_ERR_ARG;
  if (T == 0) return NSV_OK;
  if (!ids || !embed || !weight || !residual_out || !out) return NSV_ERR_ARG;
  if (rope_out && (!positions || !cos_sin || max_pos <= 0 || D <= 0)) return NSV_ERR_ARG;
  const int J = (E + kNormThreads - 1) / kNormThreads;
#define NSV_EMB(JJ)                                                                                              \
  hipLaunchKernelGGL(embed_norm_kernel<JJ>, dim3(T), dim3(kNormThreads), 0, (hipStream_t)stream, ids,           \
                     (const uint16_t*)embed, (int64_t)vocab, (const uint16_t*)weight, (uint16_t*)residual_out,  \
                     (uint16_t*)out, E, eps, positions, cos_sin, max_pos, D, rope_out)
  if (J <= 4) NSV_EMB(4);
  else if (J <= 8) NSV_EMB(8);
  else NSV_EMB(16);
#undef NSV_EMB
  return nsv_launch_status();
}

int nsv_qk_norm_rope_store(const void* qkv, const void* q_norm_w, const void* k_norm_w, const float* cos_sin,
                           int max_pos, const int64_t* positions, const int64_t* slot_mapping, void* q_out,
                           void* k_cache, void* v_cache, int T, int H, int Hkv, int D, float eps, void* stream) {
  if (T < 0 || H <= 0 || Hkv <= 0 || D <= 0 || (D & 1) || D > 128 || max_pos <= 0) return NSV_ERR_ARG;
  if (T == 0) return NSV_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !cos_sin || !slot_mapping || !q_out || !k_cache || !v_cache)
    return NSV_ERR_ARG;
  if (!positions && max_pos < T) return NSV_ERR_ARG;  // the per-row table has a row per step row
  EpilogueArgs a{(const uint16_t*)qkv, (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, cos_sin, positions,
                 slot_mapping, (uint16_t*)q_out, (uint16_t*)k_cache, (uint16_t*)v_cache, T, H, Hkv, D, max_pos, eps};
  const int64_t waves = (int64_t)T * (H + 2 * Hkv);
  if (positions)
    hipLaunchKernelGGL(qk_norm_rope_store_kernel<true>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(qk_norm_rope_store_kernel<false>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, a);
  return nsv_launch_status();
}

int nsv_silu_mul(const void* gate_up, void* out, int T, int I, void* stream) {
  if (T < 0 || I <= 0) return NSV_ERR_ARG;
  if (T == 0) return NSV_OK;
  if (!gate_up || !out) return NSV_ERR_ARG;
  const int64_t n = (int64_t)T * I;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)gate_up, (uint16_t*)out, (int64_t)T, I);
  return nsv_launch_status();
}

}  // extern "C"
