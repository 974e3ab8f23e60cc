// Acceptance step of the verification round for gfx950: greedy exact-match
// and min(1, p_t/p_d) rejection sampling with residual resampling.
//
// Behaviour follows src/myvllm/spec_engine/rejection_sampler.py:25-98 and
// the engine's batched greedy path (spec_llm_engine.py:224-243); the
// decomposition is this library's own.  Every pass over the vocabulary is
// split into chunks so that a round's rows cover the chip; per-chunk results
// go to the workspace and a small per-sequence kernel combines them.
//
// Arithmetic contract (shared with the CPU oracle): torch ops on bf16/fp32
// tensors compute in fp32 and round to the tensor dtype.  Softmax values and
// sums are the exact quantities (here: fp64 exp and fp64 accumulation)
// rounded once to fp32 and then to the dtype; quotients are IEEE fp32
// divisions rounded to the dtype; argmax takes the first index of the
// maximum with NaN as the maximum, torch's rule.  Random draws are inputs:
// torch.multinomial(p, 1) is argmax(p / q) with q ~ Exp(1) in p's dtype, and
// the uniforms of the accept test are fp32.

#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxK = 32;  // drafts per sequence the kernels handle

// ---------------------------------------------------------------------------
// element access and dtype rounding
// ---------------------------------------------------------------------------
__device__ __forceinline__ float load_elem(const void* base, int64_t i, int dtype) {
  if (dtype == NSV_BF16) return bf16_bits_to_f32(((const uint16_t*)base)[i]);
  return ((const float*)base)[i];
}

// fp32 value rounded to the dtype (bf16: round to nearest even)
__device__ __forceinline__ float round_dt(float f, int dtype) {
  if (dtype == NSV_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(f));
  return f;
}

// exact quantity (fp64) rounded to fp32, then to the dtype
__device__ __forceinline__ float round_dt_d(double x, int dtype) { return round_dt((float)x, dtype); }

// torch's a / b on dtype tensors: IEEE fp32 division rounded to the dtype
// (hipcc keeps fp32 division correctly rounded: -fhip-fp32-correctly-rounded-divide-sqrt is its default)
__device__ __forceinline__ float div_dt(float a, float b, int dtype) { return round_dt(a / b, dtype); }

// ---------------------------------------------------------------------------
// argmax as a 64-bit max: high word = the value's order-preserving bits
// (NaN above everything), low word = ~index so that ties go to the lowest
// index.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  uint32_t u = __float_as_uint(v);
  uint32_t ord;
  if (v != v) ord = 0xffffffffu;                 // NaN wins
  else if (u & 0x80000000u) ord = ~u;            // negatives: reversed
  else ord = u | 0x80000000u;                    // non-negatives above them
  if (v == 0.f) ord = 0x80000000u;               // -0 == +0
  return ((uint64_t)ord << 32) | (uint64_t)(~idx);
}
__device__ __forceinline__ uint32_t key_index(uint64_t k) { return ~(uint32_t)(k & 0xffffffffu); }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = __shfl_xor(v, o, NSV_WAVE);
    v = w > v ? w : v;
  }
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, NSV_WAVE);
  return v;
}

// workgroup reductions through a small LDS array (kThreads / 64 waves)
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  v = wave_max_u64(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  uint64_t r = red[0];
  for (int i = 1; i < kThreads / 64; ++i) r = red[i] > r ? red[i] : r;
  __syncthreads();
  return r;
}
__device__ __forceinline__ double block_sum_d(double v, double* red) {
  v = wave_sum_d(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  double r = 0.0;
  for (int i = 0; i < kThreads / 64; ++i) r += red[i];  // fixed order: deterministic
  __syncthreads();
  return r;
}
__device__ __forceinline__ float block_max_f(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

struct Chunk {
  int64_t lo, hi;
};
__device__ __forceinline__ Chunk chunk_of(int ch, int nch, int V) {
  const int64_t per = ((int64_t)V + nch - 1) / nch;
  Chunk c;
  c.lo = min((int64_t)V, ch * per);
  c.hi = min((int64_t)V, c.lo + per);
  return c;
}

// ---------------------------------------------------------------------------
// Greedy
// ---------------------------------------------------------------------------
struct GreedyArgs {
  const void* logits;
  int64_t seq_stride;  // rows between sequences
  const int32_t* drafts;
  const int32_t* num_drafts;
  int B, K, V, dtype, nch;
  uint64_t* keys;  // [B, K+1, nch]
  int32_t* out_tokens;
  int32_t* out_len;
};

// grid (B*(K+1), nch): argmax key of one chunk of one row
__global__ __launch_bounds__(kThreads) void greedy_argmax_kernel(GreedyArgs a) {
  __shared__ uint64_t red[kThreads / 64];
  const int rowid = blockIdx.x, ch = blockIdx.y;
  const int b = rowid / (a.K + 1), r = rowid - b * (a.K + 1);
  const int kb = min(max(a.num_drafts[b], 0), a.K);
  if (r > kb) return;  // uniform: a row the sequence does not use
  // chunks of a multiple of 8 elements, so that 16-byte loads stay aligned
  // (the maximum does not depend on how the row is cut)
  const int64_t per = (((int64_t)a.V + a.nch - 1) / a.nch + 7) & ~(int64_t)7;
  const int64_t base = ((int64_t)b * a.seq_stride + r) * a.V;
  uint64_t best = 0;
  int64_t lo = min((int64_t)a.V, ch * per), hi = min((int64_t)a.V, lo + per);
  if (a.dtype == NSV_BF16 && ((base + lo) & 7) == 0) {
    // 8 elements per 16-byte load, two loads in flight per iteration; the
    // rest of the chunk (fewer than 8 elements) below
    const int64_t nvec = (hi - lo) >> 3;
    const u32x4* src = reinterpret_cast<const u32x4*>((const uint16_t*)a.logits + base + lo);
    for (int64_t j = threadIdx.x; j < nvec; j += 2 * kThreads) {
      u32x4 w[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) w[u] = j + u * kThreads < nvec ? src[j + u * kThreads] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (j + u * kThreads >= nvec) break;
        const uint32_t v0 = (uint32_t)(lo + ((j + u * kThreads) << 3));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t bits = (e & 1) ? (w[u][e >> 1] >> 16) : (w[u][e >> 1] & 0xffffu);
          const uint64_t k = argmax_key(bf16_bits_to_f32(bits), v0 + e);
          best = k > best ? k : best;
        }
      }
    }
    lo += nvec << 3;
  }
  for (int64_t v = lo + threadIdx.x; v < hi; v += kThreads) {
    const uint64_t k = argmax_key(load_elem(a.logits, base + v, a.dtype), (uint32_t)v);
    best = k > best ? k : best;
  }
  best = block_max_u64(best, red);
  if (threadIdx.x == 0) a.keys[(int64_t)rowid * a.nch + ch] = best;
}

// grid B: argmax per row, then rejection_sampler.py:25-36
__global__ __launch_bounds__(64) void greedy_finalize_kernel(GreedyArgs a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int kb = min(max(a.num_drafts[b], 0), a.K);
  __shared__ int32_t amax[kMaxK + 1];
  for (int r = 0; r <= kb; ++r) {
    uint64_t best = 0;
    for (int ch = lane; ch < a.nch; ch += 64) {
      const uint64_t k = a.keys[((int64_t)b * (a.K + 1) + r) * a.nch + ch];
      best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) amax[r] = (int32_t)key_index(best);
  }
  __syncthreads();
  if (lane != 0) return;
  int n = 0;
  int32_t* out = a.out_tokens + (int64_t)b * (a.K + 1);
  for (int i = 0; i < kb; ++i) {
    const int32_t d = a.drafts[(int64_t)b * a.K + i];
    if (d != amax[i]) {
      out[n++] = amax[i];
      a.out_len[b] = n;
      return;
    }
    out[n++] = d;
  }
  out[n++] = amax[kb];  // every draft accepted: the bonus token
  a.out_len[b] = n;
}

// ---------------------------------------------------------------------------
// Stochastic
// ---------------------------------------------------------------------------
struct StochArgs {
  const void* target;        // row (b, r) at (b*t_seq + r) * V
  int64_t t_seq;
  const void* draft;         // nullable; row (b, i) at (b*d_seq + i*d_row) * V
  int64_t d_seq, d_row;
  const int32_t* drafts;     // [B, K]
  const int32_t* num_drafts; // [B]
  const float* temperature;  // [B]
  const float* uniforms;     // [B, K]
  const void* noise;         // sequence b's noise at b * q_seq: [V] (draft rows) or [K+1, V] (none)
  const int32_t* row_mode;   // nullable [B]: 0 = sequence b has no draft rows (n-gram mode)
  int64_t q_seq;
  int B, K, V, dtype, nch;
  int cdtype;                // dtype results are rounded to (the logits dtype, or fp32 for the sampler)
  int ndtype;                // dtype of the noise
  // workspace
  float* st_max;     // [B, 2K+1, nch]  chunk max of z = x / T
  double* st_sum;    // [B, 2K+1, nch]  chunk sum of exp(z - chunk max)
  uint64_t* st_key;  // [B, K+1, nch]   chunk argmax of the raw target row (greedy sequences)
  float* row_m;      // [B, 2K+1]
  double* row_s;     // [B, 2K+1]
  int32_t* dec;      // [B, 4]: row to sample (-1: none), kind (0 bonus / n-gram row, 1 resample),
                     //         accepted count, greedy flag
  int32_t* acc;      // [B, K+1] accepted prefix
  double* res_sum;   // [B, nch, 2]  chunk sums of the residual and of p_t
  uint64_t* smp_key; // [B, K+1, nch] chunk argmax of prob / q
  int32_t* out_tokens;       // sequence b's tokens at b * out_seq
  int64_t out_seq;
  int32_t* out_len;
};

__device__ __forceinline__ bool is_greedy(const StochArgs& a, int b) { return a.temperature[b] <= 1e-6f; }
// sequence b is verified against draft rows (min(1, p_t/p_d)) rather than
// by sampling every target row (n-gram drafts)
__device__ __forceinline__ bool has_rows(const StochArgs& a, int b) {
  return a.draft != nullptr && (a.row_mode == nullptr || a.row_mode[b] != 0);
}
__device__ __forceinline__ int kdrafts(const StochArgs& a, int b) {
  return a.K == 0 ? 0 : min(max(a.num_drafts[b], 0), a.K);  // K = 0: the sampler (no drafts)
}
__device__ __forceinline__ int64_t trow(const StochArgs& a, int b, int r) { return ((int64_t)b * a.t_seq + r) * a.V; }
__device__ __forceinline__ int64_t drow(const StochArgs& a, int b, int i) { return ((int64_t)b * a.d_seq + (int64_t)i * a.d_row) * a.V; }

// z = x / T rounded to the compute dtype (rejection_sampler.py:47, :52;
// layers/sampler.py:20 divides by an fp32 tensor, so there it is fp32)
__device__ __forceinline__ float scaled(const StochArgs& a, const void* base, int64_t i, float T) {
  return div_dt(load_elem(base, i, a.dtype), T, a.cdtype);
}

// softmax value round(exp(z - m) / s) of one element
__device__ __forceinline__ float prob_of(float z, float m, double s, int dtype) {
  return round_dt_d(exp((double)z - (double)m) / s, dtype);
}

// grid (B*(2K+1), nch).  Rows 0..K: target rows; K+1..2K: draft rows.
// Stochastic sequences: chunk max and sum of exp(z - max).  Greedy
// sequences: chunk argmax of the raw target row.
__global__ __launch_bounds__(kThreads) void stoch_stats_kernel(StochArgs a) {
  __shared__ float redf[kThreads / 64];
  __shared__ double redd[kThreads / 64];
  __shared__ uint64_t redk[kThreads / 64];
  const int R = 2 * a.K + 1;
  const int rowid = blockIdx.x, ch = blockIdx.y;
  const int b = rowid / R, r = rowid - b * R;
  const int kb = kdrafts(a, b);
  const bool greedy = is_greedy(a, b);
  const bool is_draft = r > a.K;
  if (!is_draft && r > kb) return;
  if (is_draft && (greedy || !has_rows(a, b) || r - a.K - 1 >= kb)) return;
  const Chunk c = chunk_of(ch, a.nch, a.V);
  const int64_t slot = (int64_t)rowid * a.nch + ch;
  if (greedy) {
    const int64_t base = trow(a, b, r);
    uint64_t best = 0;
    for (int64_t v = c.lo + threadIdx.x; v < c.hi; v += kThreads) {
      const uint64_t k = argmax_key(load_elem(a.target, base + v, a.dtype), (uint32_t)v);
      best = k > best ? k : best;
    }
    best = block_max_u64(best, redk);
    if (threadIdx.x == 0) a.st_key[((int64_t)b * (a.K + 1) + r) * a.nch + ch] = best;
    return;
  }
  const float T = a.temperature[b];
  const void* src = is_draft ? a.draft : a.target;
  const int64_t base = is_draft ? drow(a, b, r - a.K - 1) : trow(a, b, r);
  float m = -__builtin_inff();
  for (int64_t v = c.lo + threadIdx.x; v < c.hi; v += kThreads) m = fmaxf(m, scaled(a, src, base + v, T));
  m = block_max_f(m, redf);
  double s = 0.0;
  if (m != -__builtin_inff())
    for (int64_t v = c.lo + threadIdx.x; v < c.hi; v += kThreads) s += exp((double)scaled(a, src, base + v, T) - (double)m);
  s = block_sum_d(s, redd);
  if (threadIdx.x == 0) {
    a.st_max[slot] = m;
    a.st_sum[slot] = s;
  }
}

// combine the chunks of row (b, r): max M and sum of exp(z - M)
__device__ __forceinline__ void combine_row(const StochArgs& a, int b, int r, float& M, double& S) {
  const int64_t base = ((int64_t)b * (2 * a.K + 1) + r) * a.nch;
  M = -__builtin_inff();
  for (int ch = 0; ch < a.nch; ++ch) M = fmaxf(M, a.st_max[base + ch]);
  S = 0.0;
  if (M == -__builtin_inff()) return;
  for (int ch = 0; ch < a.nch; ++ch) {
    const float m = a.st_max[base + ch];
    if (m != -__builtin_inff()) S += a.st_sum[base + ch] * exp((double)m - (double)M);
  }
}

// grid B, one wave.  Row statistics; greedy sequences finish here; the
// draft-row mode walks the accept test (rejection_sampler.py:51-61) and
// picks the row to sample from.
__global__ __launch_bounds__(64) void stoch_decide_kernel(StochArgs a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int kb = kdrafts(a, b);
  const int R = 2 * a.K + 1;
  int32_t* dec = a.dec + 4 * b;
  int32_t* acc = a.acc + (int64_t)b * (a.K + 1);
  if (is_greedy(a, b)) {
    // rejection_sampler.py:95 -> verify_greedy
    __shared__ int32_t amax[kMaxK + 1];
    for (int r = 0; r <= kb; ++r) {
      uint64_t best = 0;
      for (int ch = lane; ch < a.nch; ch += 64) {
        const uint64_t k = a.st_key[((int64_t)b * (a.K + 1) + r) * a.nch + ch];
        best = k > best ? k : best;
      }
      best = wave_max_u64(best);
      if (lane == 0) amax[r] = (int32_t)key_index(best);
    }
    __syncthreads();
    if (lane == 0) {
      int n = 0;
      bool all = true;
      for (int i = 0; i < kb; ++i) {
        const int32_t d = a.drafts[(int64_t)b * a.K + i];
        if (d != amax[i]) {
          acc[n++] = amax[i];
          all = false;
          break;
        }
        acc[n++] = d;
      }
      if (all) acc[n++] = amax[kb];  // the bonus token
      dec[0] = -1;
      dec[1] = 0;
      dec[2] = n;
      dec[3] = 1;
    }
    return;
  }
  // row statistics of the rows this sequence uses
  for (int r = lane; r < R; r += 64) {
    const bool is_draft = r > a.K;
    if ((!is_draft && r > kb) || (is_draft && (!has_rows(a, b) || r - a.K - 1 >= kb))) continue;
    float M;
    double S;
    combine_row(a, b, r, M, S);
    a.row_m[(int64_t)b * R + r] = M;
    a.row_s[(int64_t)b * R + r] = S;
  }
  __syncthreads();
  if (lane != 0) return;
  dec[3] = 0;
  if (!has_rows(a, b)) {
    // n-gram mode: every row 0..kb is sampled; decisions come after
    dec[0] = kb;
    dec[1] = 0;
    dec[2] = 0;
    return;
  }
  const float T = a.temperature[b];
  const float floor = round_dt(1e-20f, a.cdtype);
  int n = 0;
  for (int i = 0; i < kb; ++i) {
    const int32_t d = a.drafts[(int64_t)b * a.K + i];
    const float pt = prob_of(scaled(a, a.target, trow(a, b, i) + d, T), a.row_m[(int64_t)b * R + i],
                             a.row_s[(int64_t)b * R + i], a.cdtype);
    const int rd = a.K + 1 + i;
    float pd = prob_of(scaled(a, a.draft, drow(a, b, i) + d, T), a.row_m[(int64_t)b * R + rd],
                       a.row_s[(int64_t)b * R + rd], a.cdtype);
    pd = fmaxf(pd, floor);                                    // clamp_min(1e-20)
    const float ratio = fminf(div_dt(pt, pd, a.cdtype), 1.0f);  // clamp(max=1)
    if (a.uniforms[(int64_t)b * a.K + i] < ratio) {
      acc[n++] = d;
      continue;
    }
    dec[0] = i;  // resample row
    dec[1] = 1;
    dec[2] = n;
    return;
  }
  dec[0] = kb;  // every draft accepted: bonus row
  dec[1] = 0;
  dec[2] = n;
}

// p_t and p_d of element v of row r (draft-row mode)
__device__ __forceinline__ void pt_pd(const StochArgs& a, int b, int r, int64_t v, float T, float& pt, float& pd) {
  const int R = 2 * a.K + 1;
  pt = prob_of(scaled(a, a.target, trow(a, b, r) + v, T), a.row_m[(int64_t)b * R + r],
               a.row_s[(int64_t)b * R + r], a.cdtype);
  const int rd = a.K + 1 + r;
  pd = prob_of(scaled(a, a.draft, drow(a, b, r) + v, T), a.row_m[(int64_t)b * R + rd],
               a.row_s[(int64_t)b * R + rd], a.cdtype);
}

// residual = max(p_t - p_d, 0) rounded to the dtype (rejection_sampler.py:63)
__device__ __forceinline__ float residual_of(float pt, float pd, int dtype) {
  return fmaxf(round_dt(pt - pd, dtype), 0.f);
}

// grid (B, nch): chunk sums of the residual and of p_t over the resample row
__global__ __launch_bounds__(kThreads) void stoch_residual_kernel(StochArgs a) {
  __shared__ double red[kThreads / 64];
  const int b = blockIdx.x, ch = blockIdx.y;
  const int32_t* dec = a.dec + 4 * b;
  if (dec[3] || dec[1] != 1) return;  // uniform: only sequences that rejected a draft
  const int r = dec[0];
  const float T = a.temperature[b];
  const Chunk c = chunk_of(ch, a.nch, a.V);
  double sr = 0.0, sp = 0.0;
  for (int64_t v = c.lo + threadIdx.x; v < c.hi; v += kThreads) {
    float pt, pd;
    pt_pd(a, b, r, v, T, pt, pd);
    sr += (double)residual_of(pt, pd, a.cdtype);
    sp += (double)pt;
  }
  sr = block_sum_d(sr, red);
  sp = block_sum_d(sp, red);
  if (threadIdx.x == 0) {
    a.res_sum[((int64_t)b * a.nch + ch) * 2 + 0] = sr;
    a.res_sum[((int64_t)b * a.nch + ch) * 2 + 1] = sp;
  }
}

// grid (B*(K+1), nch): chunk argmax of prob / q over the rows to sample
__global__ __launch_bounds__(kThreads) void stoch_sample_kernel(StochArgs a) {
  __shared__ uint64_t red[kThreads / 64];
  __shared__ float sS;
  __shared__ int sUseRes;
  const int rowid = blockIdx.x, ch = blockIdx.y;
  const int b = rowid / (a.K + 1), r = rowid - b * (a.K + 1);
  const int32_t* dec = a.dec + 4 * b;
  if (dec[3]) return;  // greedy sequence: done
  const bool ngram = !has_rows(a, b);
  if (ngram ? r > dec[0] : r != dec[0]) return;
  const int R = 2 * a.K + 1;
  const float T = a.temperature[b];
  const bool resample = !ngram && dec[1] == 1;
  if (resample) {
    if (threadIdx.x == 0) {
      double sr = 0.0, sp = 0.0;
      for (int j = 0; j < a.nch; ++j) {
        sr += a.res_sum[((int64_t)b * a.nch + j) * 2 + 0];
        sp += a.res_sum[((int64_t)b * a.nch + j) * 2 + 1];
      }
      const float Sr = round_dt_d(sr, a.cdtype);
      sUseRes = Sr > 0.f;  // rejection_sampler.py:64-65
      sS = Sr > 0.f ? Sr : round_dt_d(sp, a.cdtype);
    }
    __syncthreads();
  }
  const Chunk c = chunk_of(ch, a.nch, a.V);
  const int64_t nbase = (int64_t)b * a.q_seq + (ngram ? (int64_t)r * a.V : 0);
  uint64_t best = 0;
  for (int64_t v = c.lo + threadIdx.x; v < c.hi; v += kThreads) {
    float p;
    if (resample) {
      float pt, pd;
      pt_pd(a, b, r, v, T, pt, pd);
      p = div_dt(sUseRes ? residual_of(pt, pd, a.cdtype) : pt, sS, a.cdtype);  // :66-67 residual / sum
    } else {
      p = prob_of(scaled(a, a.target, trow(a, b, r) + v, T), a.row_m[(int64_t)b * R + r],
                  a.row_s[(int64_t)b * R + r], a.cdtype);
    }
    const float q = load_elem(a.noise, nbase + v, a.ndtype);
    const uint64_t k = argmax_key(div_dt(p, q, a.cdtype), (uint32_t)v);  // multinomial = argmax(p / q)
    best = k > best ? k : best;
  }
  best = block_max_u64(best, red);
  if (threadIdx.x == 0) a.smp_key[(int64_t)rowid * a.nch + ch] = best;
}

// grid B, one wave: sampled tokens -> accepted list
__global__ __launch_bounds__(64) void stoch_finalize_kernel(StochArgs a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int32_t* dec = a.dec + 4 * b;
  const int32_t* acc = a.acc + (int64_t)b * (a.K + 1);
  int32_t* out = a.out_tokens + (int64_t)b * a.out_seq;
  __shared__ int32_t smp[kMaxK + 1];
  const int kb = kdrafts(a, b);
  if (dec[3]) {  // greedy
    if (lane == 0) {
      for (int i = 0; i < dec[2]; ++i) out[i] = acc[i];
      a.out_len[b] = dec[2];
    }
    return;
  }
  const bool ngram = !has_rows(a, b);
  for (int r = ngram ? 0 : dec[0]; r <= dec[0]; ++r) {
    uint64_t best = 0;
    for (int ch = lane; ch < a.nch; ch += 64) {
      const uint64_t k = a.smp_key[((int64_t)b * (a.K + 1) + r) * a.nch + ch];
      best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) smp[r] = (int32_t)key_index(best);
  }
  __syncthreads();
  if (lane != 0) return;
  if (!ngram) {
    const int n = dec[2];
    for (int i = 0; i < n; ++i) out[i] = acc[i];
    out[n] = smp[dec[0]];
    a.out_len[b] = n + 1;
    return;
  }
  // rejection_sampler.py:76-85: accept while the target sample equals the draft
  int n = 0;
  for (int i = 0; i < kb; ++i) {
    const int32_t d = a.drafts[(int64_t)b * a.K + i];
    out[n++] = smp[i];
    if (smp[i] != d) {
      a.out_len[b] = n;
      return;
    }
  }
  out[n++] = smp[kb];
  a.out_len[b] = n;
}

int choose_nch(int rows, int V) {
  int nch = (512 + rows - 1) / (rows > 0 ? rows : 1);
  const int max_by_len = V / 2048 > 1 ? V / 2048 : 1;
  if (nch > max_by_len) nch = max_by_len;
  if (nch > 64) nch = 64;
  if (nch < 1) nch = 1;
  return nch;
}

size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

struct StochLayout {
  size_t st_max, st_sum, st_key, row_m, row_s, dec, acc, res_sum, smp_key, total;
};

StochLayout stoch_layout(int B, int K, int nch) {
  StochLayout L;
  const size_t R = 2 * (size_t)K + 1, K1 = (size_t)K + 1;
  size_t off = 0;
  L.st_max = off;  off += a256((size_t)B * R * nch * sizeof(float));
  L.st_sum = off;  off += a256((size_t)B * R * nch * sizeof(double));
  L.st_key = off;  off += a256((size_t)B * K1 * nch * sizeof(uint64_t));
  L.row_m = off;   off += a256((size_t)B * R * sizeof(float));
  L.row_s = off;   off += a256((size_t)B * R * sizeof(double));
  L.dec = off;     off += a256((size_t)B * 4 * sizeof(int32_t));
  L.acc = off;     off += a256((size_t)B * K1 * sizeof(int32_t));
  L.res_sum = off; off += a256((size_t)B * nch * 2 * sizeof(double));
  L.smp_key = off; off += a256((size_t)B * K1 * nch * sizeof(uint64_t));
  L.total = off;
  return L;
}

bool bad_shape(int B, int K, int V, int dtype) {
  return B < 0 || K < 0 || K > kMaxK || V <= 0 || (dtype != NSV_F32 && dtype != NSV_BF16);
}

}  // namespace

extern "C" {

size_t nsv_accept_workspace_size(int B, int K, int V, int dtype, int stochastic) {
  if (bad_shape(B, K, V, dtype)) return 0;
  if (!stochastic) return a256((size_t)B * (K + 1) * choose_nch(B * (K + 1), V) * sizeof(uint64_t));
  return stoch_layout(B, K, choose_nch(B * (2 * K + 1), V)).total;
}

int nsv_accept_greedy(const void* target_logits, int64_t seq_stride, const int32_t* drafts,
                      const int32_t* num_drafts, int B, int K, int V, int dtype, int32_t* out_tokens,
                      int32_t* out_len, void* workspace, size_t workspace_bytes, void* stream) {
  if (bad_shape(B, K, V, dtype) || seq_stride < K + 1) return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!target_logits || (!drafts && K > 0) || !num_drafts || !out_tokens || !out_len) return NSV_ERR_ARG;
  const size_t need = nsv_accept_workspace_size(B, K, V, dtype, 0);
  if (!workspace || workspace_bytes < need) return NSV_ERR_WORKSPACE;
  GreedyArgs a;
  a.logits = target_logits;
  a.seq_stride = seq_stride;
  a.drafts = drafts;
  a.num_drafts = num_drafts;
  a.B = B;
  a.K = K;
  a.V = V;
  a.dtype = dtype;
  a.nch = choose_nch(B * (K + 1), V);
  a.keys = (uint64_t*)workspace;
  a.out_tokens = out_tokens;
  a.out_len = out_len;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(greedy_argmax_kernel, dim3(B * (K + 1), a.nch), dim3(kThreads), 0, s, a);
  int rc = nsv_launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(greedy_finalize_kernel, dim3(B), dim3(64), 0, s, a);
  return nsv_launch_status();
}

}  // extern "C"

namespace {

// Fill the workspace views of `a` and launch the stochastic kernels.
int launch_stoch(StochArgs& a, const StochLayout& L, char* ws, bool any_rows, hipStream_t s) {
  a.st_max = (float*)(ws + L.st_max);
  a.st_sum = (double*)(ws + L.st_sum);
  a.st_key = (uint64_t*)(ws + L.st_key);
  a.row_m = (float*)(ws + L.row_m);
  a.row_s = (double*)(ws + L.row_s);
  a.dec = (int32_t*)(ws + L.dec);
  a.acc = (int32_t*)(ws + L.acc);
  a.res_sum = (double*)(ws + L.res_sum);
  a.smp_key = (uint64_t*)(ws + L.smp_key);
  const int B = a.B, K = a.K, nch = a.nch;
  hipLaunchKernelGGL(stoch_stats_kernel, dim3(B * (2 * K + 1), nch), dim3(kThreads), 0, s, a);
  int rc = nsv_launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(stoch_decide_kernel, dim3(B), dim3(64), 0, s, a);
  if ((rc = nsv_launch_status())) return rc;
  if (any_rows) {
    hipLaunchKernelGGL(stoch_residual_kernel, dim3(B, nch), dim3(kThreads), 0, s, a);
    if ((rc = nsv_launch_status())) return rc;
  }
  hipLaunchKernelGGL(stoch_sample_kernel, dim3(B * (K + 1), nch), dim3(kThreads), 0, s, a);
  if ((rc = nsv_launch_status())) return rc;
  hipLaunchKernelGGL(stoch_finalize_kernel, dim3(B), dim3(64), 0, s, a);
  return nsv_launch_status();
}

}  // namespace

extern "C" {

int nsv_accept_stochastic(const void* target_logits, int64_t target_seq_stride, const void* draft_logits,
                          int64_t draft_seq_stride, int64_t draft_row_stride, const int32_t* draft_mode,
                          const int32_t* drafts, const int32_t* num_drafts, const float* temperature,
                          const float* uniforms, const void* noise, int64_t noise_seq_stride, int B, int K, int V,
                          int dtype, int32_t* out_tokens, int32_t* out_len, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (bad_shape(B, K, V, dtype) || target_seq_stride < K + 1) return NSV_ERR_ARG;
  if (draft_logits && (draft_row_stride < 1 || draft_seq_stride < 0)) return NSV_ERR_ARG;
  if (draft_mode && !draft_logits) return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!target_logits || (!drafts && K > 0) || !num_drafts || !temperature || !noise || !out_tokens || !out_len)
    return NSV_ERR_ARG;
  if (draft_logits && !uniforms && K > 0) return NSV_ERR_ARG;
  // noise per sequence: [V] when every sequence has draft rows, else [K+1, V]
  const int64_t q_default = (draft_logits && !draft_mode) ? (int64_t)V : (int64_t)(K + 1) * V;
  if (noise_seq_stride == 0) noise_seq_stride = q_default;
  if (noise_seq_stride < q_default) return NSV_ERR_ARG;
  const int nch = choose_nch(B * (2 * K + 1), V);
  const StochLayout L = stoch_layout(B, K, nch);
  if (!workspace || workspace_bytes < L.total) return NSV_ERR_WORKSPACE;
  StochArgs a;
  a.target = target_logits;
  a.t_seq = target_seq_stride;
  a.draft = draft_logits;
  a.d_seq = draft_seq_stride;
  a.d_row = draft_row_stride;
  a.drafts = drafts;
  a.num_drafts = num_drafts;
  a.temperature = temperature;
  a.uniforms = uniforms;
  a.noise = noise;
  a.row_mode = draft_mode;
  a.q_seq = noise_seq_stride;
  a.B = B;
  a.K = K;
  a.V = V;
  a.dtype = dtype;
  a.cdtype = dtype;
  a.ndtype = dtype;
  a.nch = nch;
  a.out_tokens = out_tokens;
  a.out_seq = K + 1;
  a.out_len = out_len;
  return launch_stoch(a, L, (char*)workspace, draft_logits != nullptr, (hipStream_t)stream);
}

size_t nsv_sample_workspace_size(int B, int V, int dtype) {
  if (bad_shape(B, 0, V, dtype)) return 0;
  return stoch_layout(B, 0, choose_nch(B, V)).total + a256((size_t)B * sizeof(int32_t));
}

int nsv_sample(const void* logits, int64_t row_stride, const float* temperature, const float* noise, int B, int V,
               int dtype, int32_t* out_tokens, int64_t out_stride, void* workspace, size_t workspace_bytes,
               void* stream) {
  if (bad_shape(B, 0, V, dtype) || row_stride < V || row_stride % V || out_stride < 1) return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!logits || !temperature || !noise || !out_tokens) return NSV_ERR_ARG;
  const int nch = choose_nch(B, V);
  const StochLayout L = stoch_layout(B, 0, nch);
  if (!workspace || workspace_bytes < nsv_sample_workspace_size(B, V, dtype)) return NSV_ERR_WORKSPACE;
  StochArgs a;
  a.target = logits;
  a.t_seq = row_stride / V;
  a.draft = nullptr;
  a.d_seq = 0;
  a.d_row = 1;
  a.drafts = nullptr;
  a.num_drafts = nullptr;
  a.temperature = temperature;
  a.uniforms = nullptr;
  a.noise = noise;
  a.row_mode = nullptr;
  a.q_seq = V;
  a.B = B;
  a.K = 0;
  a.V = V;
  a.dtype = dtype;
  a.cdtype = NSV_F32;  // logits / (fp32 tensor) promotes to fp32 (layers/sampler.py:20-23)
  a.ndtype = NSV_F32;
  a.nch = nch;
  a.out_tokens = out_tokens;
  a.out_seq = out_stride;
  a.out_len = (int32_t*)((char*)workspace + L.total);
  return launch_stoch(a, L, (char*)workspace, false, (hipStream_t)stream);
}

}  // extern "C"
