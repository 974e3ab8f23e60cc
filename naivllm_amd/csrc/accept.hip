// Acceptance step of the verification round for gfx950: greedy exact-match
// and min(1, p_t/p_d) rejection sampling with residual resampling.
//
// Behaviour follows src/myvllm/spec_engine/rejection_sampler.py:25-98 and
// the engine's batched greedy path (spec_llm_engine.py:224-243); the
// decomposition is this library's own.  Every pass over the vocabulary is
// split into chunks so that a round's rows cover the chip; each workgroup
// holds its chunk in registers (16-byte loads, all issued before any is
// used), so a row is read from HBM once per pass.  Per-chunk results go to
// the workspace and a per-sequence kernel combines them, every entry loaded
// in one round trip:
//   greedy      chunk argmax keys | walk
//   stochastic  chunk (max, sum exp) of every row | accept walk |
//               residual sums of the resampled row (model drafts) |
//               chunk argmax of prob / q | output tokens
// (Combining in the last workgroup to finish, behind an arrival counter per
// sequence, was measured slower: a few hundred same-address device-scope
// atomics per sequence serialise at ~20 ns each, far above a launch gap.)
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
#include "exp_f64.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxK = 63;  // drafts per sequence: K+1 rows fit one 64-lane ballot
// row-statistics / argmax pass: a chunk is read in slabs of kThreads*EPT
// elements, EPT per thread held in registers (EPT = 32, or 8 when few rows
// would leave the chip idle); at most kMaxChunks chunks per row (longer
// chunks take several slabs)
constexpr int kEptWide = 32;
constexpr int kEptNarrow = 8;
constexpr int kMaxChunks = 128;
// residual / sample pass (one or a few rows per sequence): smaller chunks
constexpr int kEpt2 = 8;
constexpr int kChunk2 = kThreads * kEpt2;
// rows per wave whose chunk entries are loaded in one round trip when a
// sequence's rows are combined
constexpr int kRowsPerWave = 9;

// ---------------------------------------------------------------------------
// element access and dtype rounding
// ---------------------------------------------------------------------------
template <typename T> struct Elem;
template <> struct Elem<uint16_t> {  // bf16 bits
  __device__ static float get(uint16_t v) { return bf16_bits_to_f32(v); }
  __device__ static float unpack(const u32x4& w, int e) {
    return bf16_bits_to_f32((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
  }
};
template <> struct Elem<float> {
  __device__ static float get(float v) { return v; }
  __device__ static float unpack(const u32x4& w, int e) { return __uint_as_float(w[e]); }
};

// fp32 value rounded to the dtype (bf16: round to nearest even)
__device__ __forceinline__ float round_dt(float f, int dtype) {
  if (dtype == NSV_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(f));
  return f;
}

// fp64 quantity rounded to fp32, then to the dtype
__device__ __forceinline__ float round_dt_d(double x, int dtype) { return round_dt((float)x, dtype); }

// torch's a / b on dtype tensors: IEEE fp32 division rounded to the dtype
// (hipcc keeps fp32 division correctly rounded: -fhip-fp32-correctly-rounded-divide-sqrt is its default)
__device__ __forceinline__ float div_dt(float a, float b, int dtype) { return round_dt(a / b, dtype); }

// the fp64 exp table, copied into LDS by a workgroup's 256 threads, one
// entry each (visible after the workgroup's next barrier)
static_assert(kThreads >= 256, "one thread per exp table entry");
__device__ __forceinline__ void load_exp_table(double* tab) {
  if (threadIdx.x < 256) tab[threadIdx.x] = kExp2Frac256[threadIdx.x];
}

// softmax value of one element: exp(z - m) * (1 / s) in fp64 (within a few
// fp64 ulps of the exact quotient), rounded to fp32 and then to the dtype
__device__ __forceinline__ float prob_of(float z, float m, double inv_s, int dtype, const double* tab) {
  return round_dt_d(nsv_exp_nonpos((double)z - (double)m, tab) * inv_s, dtype);
}

// ---------------------------------------------------------------------------
// a slab of a row in registers: x[j] holds element slab_index(lo, j) for
// indices below hi and -inf past it.  Thread t holds groups of kGroup
// consecutive elements, group g at lo + kGroup*(t + g*kThreads), so every
// row of a kernel (logits of either dtype, noise) shares one element order;
// a 16-byte aligned row is read with 16-byte loads, any other element by
// element.
// ---------------------------------------------------------------------------
constexpr int kGroup = 8;

__device__ __forceinline__ int64_t slab_index(int64_t lo, int j) {
  return lo + (int64_t)kGroup * (threadIdx.x + (j / kGroup) * kThreads) + (j % kGroup);
}

template <typename T>
__device__ __forceinline__ bool aligned16(const T* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

template <typename T, int EPT>
__device__ __forceinline__ void load_slab(const T* row, int64_t lo, int64_t hi, float (&x)[EPT]) {
  constexpr int PER = 16 / sizeof(T);       // elements per 16-byte load
  constexpr int L = kGroup / PER;           // loads per group
  constexpr int G = EPT / kGroup;           // groups per thread
  static_assert(EPT % kGroup == 0 && kGroup % PER == 0, "slab shape");
  if (aligned16(row)) {  // lo is a multiple of kGroup: group starts stay aligned
    u32x4 w[G][L];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t v0 = slab_index(lo, g * kGroup);
#pragma unroll
      for (int l = 0; l < L; ++l)
        w[g][l] = v0 + kGroup <= hi ? load16_stream(row + v0 + l * PER) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t v0 = slab_index(lo, g * kGroup);
      const bool whole = v0 + kGroup <= hi;
#pragma unroll
      for (int e = 0; e < kGroup; ++e) {
        float f = Elem<T>::unpack(w[g][e / PER], e % PER);
        if (!whole) f = v0 + e < hi ? Elem<T>::get(row[v0 + e]) : -__builtin_inff();  // the row's ragged end
        x[g * kGroup + e] = f;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int64_t v = slab_index(lo, j);
      x[j] = v < hi ? Elem<T>::get(row[v]) : -__builtin_inff();
    }
  }
}

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

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) { return wave_max_u64_dpp(v); }
__device__ __forceinline__ double wave_sum_d(double v) { return wave_sum_dpp(v); }
__device__ __forceinline__ float wave_max_f(float v) { return wave_max_dpp(v); }

// workgroup reductions through a small LDS array (one slot per wave)
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* red) {
  v = wave_max_u64(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  uint64_t r = red[0];
  for (int i = 1; i < kWaves; ++i) r = red[i] > r ? red[i] : r;
  __syncthreads();
  return r;
}
__device__ __forceinline__ double block_sum_d(double v, double* red) {
  v = wave_sum_d(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  double r = 0.0;
  for (int i = 0; i < kWaves; ++i) r += red[i];  // fixed order: deterministic
  __syncthreads();
  return r;
}
// two sums through one exchange (each summed as block_sum_d sums it)
__device__ __forceinline__ void block_sum2_d(double& u, double& v, double* red) {
  u = wave_sum_d(u);
  v = wave_sum_d(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    red[w] = u;
    red[kWaves + w] = v;
  }
  __syncthreads();
  double ru = 0.0, rv = 0.0;
  for (int i = 0; i < kWaves; ++i) {  // fixed order: deterministic
    ru += red[i];
    rv += red[kWaves + i];
  }
  __syncthreads();
  u = ru;
  v = rv;
}
__device__ __forceinline__ float block_max_f(float v, float* red) {
  v = wave_max_f(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kWaves; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

// chunking of the row-statistics pass: nch chunks of `per` elements (a
// multiple of 8, so chunk starts keep 16-byte alignment)
struct Chunk {
  int64_t lo, hi;
};
__device__ __forceinline__ Chunk chunk_of(int ch, int nch, int V) {
  const int64_t per = (((int64_t)V + nch - 1) / nch + 7) & ~(int64_t)7;
  Chunk c;
  c.lo = min((int64_t)V, ch * per);
  c.hi = min((int64_t)V, c.lo + per);
  return c;
}
__device__ __forceinline__ Chunk chunk2_of(int ch, int V) {
  Chunk c;
  c.lo = min((int64_t)V, (int64_t)ch * kChunk2);
  c.hi = min((int64_t)V, c.lo + kChunk2);
  return c;
}

// First index of the maximum of a thread's slab values (NaN above every
// number and the first NaN wins, -0 == +0, torch's argmax), as the argmax
// key of that element; 0 when every slot lies past hi.  Slot order is index
// order, so a strict comparison keeps the first of equal values.
template <int EPT>
__device__ __forceinline__ uint64_t thread_argmax(const float (&x)[EPT], int64_t lo, int64_t hi) {
  float best = x[0];
  int bj = 0;
  bool nan = x[0] != x[0];
#pragma unroll
  for (int j = 1; j < EPT; ++j) {
    const bool gt = x[j] > best;
    best = gt ? x[j] : best;
    bj = gt ? j : bj;
    nan |= x[j] != x[j];
  }
  if (nan) {
#pragma unroll
    for (int j = EPT - 1; j >= 0; --j)
      if (x[j] != x[j]) {
        best = x[j];
        bj = j;
      }
  }
  const int64_t v = slab_index(lo, bj);
  return v < hi ? argmax_key(best, (uint32_t)v) : 0ull;
}

// argmax key of a thread's elements of chunk c of a row (several slabs
// when the chunk is longer than kThreads*EPT)
template <typename T, int EPT>
__device__ __forceinline__ uint64_t chunk_argmax(const T* row, const Chunk& c) {
  uint64_t best = 0;
  for (int64_t lo = c.lo; lo < c.hi; lo += (int64_t)kThreads * EPT) {
    float x[EPT];
    load_slab<T, EPT>(row, lo, c.hi, x);
    const uint64_t k = thread_argmax<EPT>(x, lo, c.hi);
    best = k > best ? k : best;
  }
  return best;
}

// ---------------------------------------------------------------------------
// Greedy walk (rejection_sampler.py:25-36) of one sequence over its
// per-chunk argmax keys [K+1][nch] (one workgroup).  Every key and draft is
// loaded before kb is needed, so the walk costs one round trip.
// ---------------------------------------------------------------------------
__device__ void greedy_walk(const uint64_t* keys, int nch, int K, int kb, const int32_t* drafts, int32_t* out,
                            int32_t* out_len) {
  __shared__ uint64_t sKey[kMaxK + 1];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int32_t d = lane < K ? drafts[lane] : 0;
  for (int r0 = 0; r0 <= K; r0 += kWaves * kRowsPerWave) {
    uint64_t k[kRowsPerWave][2];
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) {
      const int r = r0 + w + j * kWaves;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = lane + 64 * h;
        k[j][h] = (r <= K && c < nch) ? keys[(int64_t)r * nch + c] : 0ull;
      }
    }
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) {
      const int r = r0 + w + j * kWaves;
      const uint64_t m = wave_max_u64(k[j][0] > k[j][1] ? k[j][0] : k[j][1]);
      if (r <= K && lane == 0) sKey[r] = m;
    }
  }
  __syncthreads();
  if (w != 0) return;
  const int32_t amax = lane <= kb ? (int32_t)key_index(sKey[lane]) : 0;
  const uint64_t miss = __ballot(lane < kb && d != amax);
  const int n = miss ? __ffsll((long long)miss) - 1 : kb;  // drafts accepted
  if (lane < n) out[lane] = d;
  if (lane == n) out[n] = amax;  // the correction, or the bonus token
  if (lane == 0) *out_len = n + 1;
}

// ---------------------------------------------------------------------------
// Greedy
// ---------------------------------------------------------------------------
struct GreedyArgs {
  const void* logits;
  int64_t seq_stride;  // rows between sequences
  const int32_t* drafts;
  const int32_t* num_drafts;
  int B, K, V, nch;
  uint64_t* keys;  // [B, K+1, nch]
  int32_t* out_tokens;
  int32_t* out_len;
};

// grid (B*(K+1), nch): argmax key of one chunk of one row
template <typename T, int EPT>
__global__ __launch_bounds__(kThreads) void greedy_argmax_kernel(GreedyArgs a) {
  __shared__ uint64_t red[kWaves];
  const int rowid = blockIdx.x, ch = blockIdx.y;
  const int b = rowid / (a.K + 1), r = rowid - b * (a.K + 1);
  const int kb = min(max(a.num_drafts[b], 0), a.K);
  if (r > kb) return;  // uniform: a row the sequence does not use
  const T* row = (const T*)a.logits + ((int64_t)b * a.seq_stride + r) * a.V;
  const uint64_t best = block_max_u64(chunk_argmax<T, EPT>(row, chunk_of(ch, a.nch, a.V)), red);
  if (threadIdx.x == 0) a.keys[(int64_t)rowid * a.nch + ch] = best;
}

// grid B: the walk of each sequence
__global__ __launch_bounds__(kThreads) void greedy_finalize_kernel(GreedyArgs a) {
  const int b = blockIdx.x;
  const int nd = a.num_drafts[b];
  greedy_walk(a.keys + (int64_t)b * (a.K + 1) * a.nch, a.nch, a.K, min(max(nd, 0), a.K), a.drafts + (int64_t)b * a.K,
              a.out_tokens + (int64_t)b * (a.K + 1), a.out_len + b);
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
  const float* uniforms;     // [B, K] (nullable without draft rows)
  const void* noise;         // sequence b's noise at b * q_seq: [V] (draft rows) or [K+1, V] (none)
  const int32_t* row_mode;   // nullable [B]: 0 = sequence b has no draft rows (n-gram mode)
  int64_t q_seq;
  int B, K, V;
  int rows;                  // statistics rows per sequence in the grid: 2K+1 with draft rows, else K+1
  int nch;                   // chunks per row of the statistics pass
  int nch2;                  // chunks per row of the residual / sample passes
  int cdtype;                // dtype results are rounded to (the logits dtype, or fp32 for the sampler)
  // workspace
  float* st_max;       // [B, 2K+1, nch]  chunk max of z = x / T
  double* st_sum;      // [B, 2K+1, nch]  chunk sum of exp(z - chunk max)
  uint64_t* st_key;    // [B, K+1, nch]   chunk argmax of the raw target row (greedy sequences)
  float* zpos;         // [B, 2K+1]       z at the row's draft token (rows 0..K-1, K+1..2K)
  float* row_m;        // [B, 2K+1]
  double* row_s;       // [B, 2K+1]
  int32_t* dec;        // [B, 4]: row to sample, kind (0 bonus / n-gram rows, 1 resample),
                       //         accepted count, greedy flag (sequence already finished)
  int32_t* acc;        // [B, K+1] accepted prefix
  double* res_part;    // [B, nch2, 2]  chunk sums of the residual and of p_t
  uint64_t* smp_key;   // [B, K+1, nch2] chunk argmax of prob / q
  int32_t* out_tokens; // sequence b's tokens at b * out_seq
  int64_t out_seq;
  int32_t* out_len;
};

__device__ __forceinline__ bool greedy_t(float T) { return T <= 1e-6f; }
__device__ __forceinline__ bool is_greedy(const StochArgs& a, int b) { return greedy_t(a.temperature[b]); }
// sequence b is verified against draft rows (min(1, p_t/p_d)) rather than
// by sampling every target row (n-gram drafts)
__device__ __forceinline__ bool has_rows(const StochArgs& a, int b) {
  return a.draft != nullptr && (a.row_mode == nullptr || a.row_mode[b] != 0);
}
__device__ __forceinline__ int kdrafts(const StochArgs& a, int b) {
  return a.K == 0 ? 0 : min(max(a.num_drafts[b], 0), a.K);  // K = 0: the sampler (no drafts)
}
__device__ __forceinline__ int64_t trow(const StochArgs& a, int b, int r) { return ((int64_t)b * a.t_seq + r) * a.V; }
__device__ __forceinline__ int64_t drow(const StochArgs& a, int b, int i) {
  return ((int64_t)b * a.d_seq + (int64_t)i * a.d_row) * a.V;
}

// z = x / T rounded to the compute dtype (rejection_sampler.py:47, :52;
// layers/sampler.py:20 divides by an fp32 tensor, so there it is fp32).
// x / 1 is x, already representable in both dtypes.
__device__ __forceinline__ float scale_by(float x, float T, bool unit, int cdtype) {
  return unit ? x : div_dt(x, T, cdtype);
}

// grid (B*rows, nch).  Rows 0..K: target rows; K+1..2K: draft rows.
// Stochastic sequences: chunk max and sum of exp(z - max), and z at the
// row's draft token when this chunk holds it.  Greedy sequences: chunk
// argmax of the raw target row.
template <typename T, int EPT>
__global__ __launch_bounds__(kThreads) void stoch_stats_kernel(StochArgs a) {
  __shared__ float redf[kWaves];
  __shared__ double redd[kWaves];
  __shared__ uint64_t redk[kWaves];
  __shared__ double etab[256];
  constexpr int SLAB = kThreads * EPT;
  const int R = 2 * a.K + 1;
  const int rowid = blockIdx.x, ch = blockIdx.y;
  const int b = rowid / a.rows, r = rowid - b * a.rows;
  const int kb = kdrafts(a, b);
  const bool greedy = is_greedy(a, b);
  const bool is_draft = r > a.K;
  const int i = is_draft ? r - a.K - 1 : r;  // draft index of the row
  // the row's draft token (loaded with the metadata; the accept test needs its z)
  const int32_t dtok = i < a.K ? a.drafts[(int64_t)b * a.K + i] : -1;
  const bool rows = has_rows(a, b);
  const bool active = is_draft ? (!greedy && rows && i < kb) : r <= kb;
  if (!active) return;  // uniform
  const Chunk c = chunk_of(ch, a.nch, a.V);
  const int64_t slot = ((int64_t)b * R + r) * a.nch + ch;
  if (greedy) {
    const T* row = (const T*)a.target + trow(a, b, r);
    const uint64_t best = block_max_u64(chunk_argmax<T, EPT>(row, c), redk);
    if (threadIdx.x == 0) a.st_key[((int64_t)b * (a.K + 1) + r) * a.nch + ch] = best;
    return;
  }
  load_exp_table(etab);
  const float Tb = a.temperature[b];
  const bool unit = Tb == 1.0f;
  const T* row = (const T*)(is_draft ? a.draft : a.target) + (is_draft ? drow(a, b, i) : trow(a, b, r));
  // z at the draft token (draft rows, and target rows before the bonus row):
  // the chunk that holds it reads it with its slab
  const int32_t d = rows && i < kb ? dtok : -1;
  const bool own_d = threadIdx.x == 0 && d >= c.lo && d < c.hi;
  const float xd = own_d ? Elem<T>::get(row[d]) : 0.f;
  // running max over the chunk's slabs (one slab when the chunk fits);
  // each thread's sum is rescaled when the max grows
  float m = -__builtin_inff();
  double s = 0.0;
  bool nan = false;
  for (int64_t lo = c.lo; lo < c.hi; lo += SLAB) {
    float z[EPT];
    load_slab<T, EPT>(row, lo, c.hi, z);
    float ms = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      z[j] = scale_by(z[j], Tb, unit, a.cdtype);
      ms = fmaxf(ms, z[j]);
      nan |= z[j] != z[j];
    }
    const float mn = fmaxf(m, block_max_f(ms, redf));  // its barrier also publishes etab
    if (mn == -__builtin_inff()) continue;
    if (m != -__builtin_inff() && mn != m) s *= nsv_exp_nonpos((double)m - (double)mn, etab);
    m = mn;
    const double md = (double)m;
#pragma unroll
    for (int j = 0; j < EPT; ++j) s += nsv_exp_nonpos((double)z[j] - md, etab);  // past-the-end slots: -inf -> 0
  }
  if (nan && m != -__builtin_inff()) s = __builtin_nan("");
  s = block_sum_d(s, redd);
  if (threadIdx.x == 0) {
    a.st_max[slot] = m;
    a.st_sum[slot] = s;
    if (own_d) a.zpos[(int64_t)b * R + r] = scale_by(xd, Tb, unit, a.cdtype);
  }
}

// grid B: the accept walk of sequence b (rejection_sampler.py:51-61).
// Combines the chunk statistics of every row into (max, sum), then decides
// every draft at once and keeps the prefix before the first rejection.
// Everything a stochastic sequence needs is loaded in one round trip,
// before its metadata is known (rows it does not use are combined and
// ignored).
__global__ __launch_bounds__(kThreads) void stoch_decide_kernel(StochArgs a) {
  __shared__ float sM[2 * kMaxK + 1];
  __shared__ double sS[2 * kMaxK + 1];
  __shared__ double etab[256];
  const int b = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int K = a.K, R = 2 * K + 1, nch = a.nch;
  const int nrows = a.rows;  // the rows the statistics pass may have written
  load_exp_table(etab);
  const float Tb = a.temperature[b];
  const int nd = K == 0 ? 0 : a.num_drafts[b];
  const bool rows = has_rows(a, b);
  int32_t d = 0;
  float u = 0.f, zt = -__builtin_inff(), zd = -__builtin_inff();
  if (lane < K) {
    d = a.drafts[(int64_t)b * K + lane];
    if (a.uniforms) u = a.uniforms[(int64_t)b * K + lane];
    zt = a.zpos[(int64_t)b * R + lane];
    if (a.draft) zd = a.zpos[(int64_t)b * R + K + 1 + lane];
  }
  const int kb = min(max(nd, 0), K);
  int32_t* dec = a.dec + 4 * b;
  // row q of the grid's row list is storage row q (target 0..K, draft K+1..2K);
  // the first batch of rows is loaded with the metadata above, before the
  // greedy test (a barrier would wait for every load in flight)
  for (int q0 = 0; q0 < nrows; q0 += kWaves * kRowsPerWave) {
    float m[kRowsPerWave][2];
    double s[kRowsPerWave][2];
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) {
      const int q = q0 + w + j * kWaves;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = lane + 64 * h;
        const bool ok = q < nrows && c < nch;
        const int64_t e = ((int64_t)b * R + q) * nch + c;
        m[j][h] = ok ? a.st_max[e] : -__builtin_inff();
        s[j][h] = ok ? a.st_sum[e] : 0.0;
      }
    }
    if (greedy_t(Tb)) break;  // uniform
    __syncthreads();  // etab
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) {
      const int q = q0 + w + j * kWaves;
      const float M = wave_max_f(fmaxf(m[j][0], m[j][1]));
      // chunks with no finite element hold sum 0 and are skipped
      double t = 0.0;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (m[j][h] != -__builtin_inff()) t += s[j][h] * nsv_exp_nonpos((double)m[j][h] - (double)M, etab);
      double S = wave_sum_d(t);
      if (M == -__builtin_inff()) S = 0.0;
      if (q < nrows && lane == 0) {
        sM[q] = M;
        sS[q] = S;
        a.row_m[(int64_t)b * R + q] = M;
        a.row_s[(int64_t)b * R + q] = S;
      }
    }
  }
  if (greedy_t(Tb)) {  // rejection_sampler.py:95 -> verify_greedy; finished here
    greedy_walk(a.st_key + (int64_t)b * (K + 1) * nch, nch, K, kb, a.drafts + (int64_t)b * K,
                a.out_tokens + (int64_t)b * a.out_seq, a.out_len + b);
    if (tid == 0) dec[3] = 1;
    return;
  }
  __syncthreads();
  if (w != 0) return;
  if (!rows) {  // n-gram mode: every row 0..kb is sampled; decisions come after
    if (lane == 0) {
      dec[0] = kb;
      dec[1] = 0;
      dec[2] = 0;
      dec[3] = 0;
    }
    return;
  }
  // lane i decides draft i: u_i < min(1, p_t(d_i) / max(p_d(d_i), 1e-20))
  const int i = lane;
  bool reject = false;
  if (i < kb) {
    if (d < 0 || d >= a.V) zt = zd = -__builtin_inff();  // a token outside the vocabulary has probability 0
    const float pt = prob_of(zt, sM[i], 1.0 / sS[i], a.cdtype, etab);
    float pd = prob_of(zd, sM[K + 1 + i], 1.0 / sS[K + 1 + i], a.cdtype, etab);
    pd = fmaxf(pd, round_dt(1e-20f, a.cdtype));                 // clamp_min(1e-20)
    const float ratio = fminf(div_dt(pt, pd, a.cdtype), 1.0f);  // clamp(max=1)
    reject = !(u < ratio);
  }
  const uint64_t rej = __ballot(reject);
  const int n = rej ? __ffsll((long long)rej) - 1 : kb;  // drafts accepted
  if (i < n) a.acc[(int64_t)b * (K + 1) + i] = d;
  if (lane == 0) {
    dec[0] = n;               // the resample row, or kb: the bonus row
    dec[1] = n < kb ? 1 : 0;
    dec[2] = n;
    dec[3] = 0;
  }
}

// residual = max(p_t - p_d, 0) rounded to the dtype (rejection_sampler.py:63)
__device__ __forceinline__ float residual_of(float pt, float pd, int dtype) {
  return fmaxf(round_dt(pt - pd, dtype), 0.f);
}

// grid (B, nch2): chunk sums of the residual and of p_t over the resample
// row of sequences that rejected a draft
template <typename T>
__global__ __launch_bounds__(kThreads) void stoch_residual_kernel(StochArgs a) {
  __shared__ double red[2 * kWaves];
  __shared__ double etab[256];
  const int b = blockIdx.x, ch = blockIdx.y;
  const int32_t* dec = a.dec + 4 * b;
  if (dec[3] || dec[1] != 1) return;  // uniform: only sequences that rejected a draft
  load_exp_table(etab);
  const int r = dec[0], R = 2 * a.K + 1;
  const float Tb = a.temperature[b];
  const bool unit = Tb == 1.0f;
  const Chunk c = chunk2_of(ch, a.V);
  float xt[kEpt2], xd[kEpt2];
  load_slab<T, kEpt2>((const T*)a.target + trow(a, b, r), c.lo, c.hi, xt);
  load_slab<T, kEpt2>((const T*)a.draft + drow(a, b, r), c.lo, c.hi, xd);
  const float mt = a.row_m[(int64_t)b * R + r], md = a.row_m[(int64_t)b * R + a.K + 1 + r];
  const double it = 1.0 / a.row_s[(int64_t)b * R + r], id = 1.0 / a.row_s[(int64_t)b * R + a.K + 1 + r];
  __syncthreads();  // etab
  double sr = 0.0, sp = 0.0;
#pragma unroll
  for (int j = 0; j < kEpt2; ++j) {
    if (slab_index(c.lo, j) >= c.hi) continue;
    const float pt = prob_of(scale_by(xt[j], Tb, unit, a.cdtype), mt, it, a.cdtype, etab);
    const float pd = prob_of(scale_by(xd[j], Tb, unit, a.cdtype), md, id, a.cdtype, etab);
    sr += (double)residual_of(pt, pd, a.cdtype);
    sp += (double)pt;
  }
  block_sum2_d(sr, sp, red);
  if (threadIdx.x == 0) {
    a.res_part[((int64_t)b * a.nch2 + ch) * 2 + 0] = sr;
    a.res_part[((int64_t)b * a.nch2 + ch) * 2 + 1] = sp;
  }
}

// grid (B, nch2, K+1 or 1): chunk argmax of prob / q over the rows to
// sample (z = 0: the resample / bonus row of a sequence with draft rows;
// z = r: row r of an n-gram sequence)
template <typename T, typename TQ>
__global__ __launch_bounds__(kThreads) void stoch_sample_kernel(StochArgs a) {
  __shared__ uint64_t red[kWaves];
  __shared__ double redd[2 * kWaves];
  __shared__ double etab[256];
  const int b = blockIdx.x, ch = blockIdx.y, j = blockIdx.z;
  const int32_t* dec = a.dec + 4 * b;
  if (dec[3]) return;  // greedy sequence: finished by the accept walk
  const bool ngram = !has_rows(a, b);
  const int last_row = dec[0];
  if (ngram ? j > last_row : j != 0) return;
  load_exp_table(etab);
  const int r = ngram ? j : last_row;
  const int R = 2 * a.K + 1;
  const float Tb = a.temperature[b];
  const bool unit = Tb == 1.0f;
  const bool resample = !ngram && dec[1] == 1;
  const Chunk c = chunk2_of(ch, a.V);
  float xt[kEpt2], xq[kEpt2];
  load_slab<T, kEpt2>((const T*)a.target + trow(a, b, r), c.lo, c.hi, xt);
  load_slab<TQ, kEpt2>((const TQ*)a.noise + (int64_t)b * a.q_seq + (ngram ? (int64_t)r * a.V : 0), c.lo, c.hi, xq);
  const float mt = a.row_m[(int64_t)b * R + r];
  const double it = 1.0 / a.row_s[(int64_t)b * R + r];
  float p[kEpt2];
  if (resample) {
    float xd[kEpt2];
    load_slab<T, kEpt2>((const T*)a.draft + drow(a, b, r), c.lo, c.hi, xd);
    const float md = a.row_m[(int64_t)b * R + a.K + 1 + r];
    const double id = 1.0 / a.row_s[(int64_t)b * R + a.K + 1 + r];
    // the divisor (rejection_sampler.py:63-67): the residual sum, or p_t's
    // when it is 0; every chunk of the row folds the chunk sums in one order
    double tr = 0.0, tp = 0.0;
    for (int k = threadIdx.x; k < a.nch2; k += kThreads) {
      tr += a.res_part[((int64_t)b * a.nch2 + k) * 2 + 0];
      tp += a.res_part[((int64_t)b * a.nch2 + k) * 2 + 1];
    }
    block_sum2_d(tr, tp, redd);  // its barriers also publish etab
    const float Sr = round_dt_d(tr, a.cdtype);
    const bool use_res = Sr > 0.f;
    const float S = use_res ? Sr : round_dt_d(tp, a.cdtype);
#pragma unroll
    for (int e = 0; e < kEpt2; ++e) {
      const float pt = prob_of(scale_by(xt[e], Tb, unit, a.cdtype), mt, it, a.cdtype, etab);
      const float pd = prob_of(scale_by(xd[e], Tb, unit, a.cdtype), md, id, a.cdtype, etab);
      p[e] = div_dt(use_res ? residual_of(pt, pd, a.cdtype) : pt, S, a.cdtype);  // :66-67 residual / sum
    }
  } else {
    __syncthreads();  // etab
#pragma unroll
    for (int e = 0; e < kEpt2; ++e) p[e] = prob_of(scale_by(xt[e], Tb, unit, a.cdtype), mt, it, a.cdtype, etab);
  }
  // multinomial = argmax(p / q); slots past the row's end never win
#pragma unroll
  for (int e = 0; e < kEpt2; ++e)
    p[e] = slab_index(c.lo, e) < c.hi ? div_dt(p[e], xq[e], a.cdtype) : -__builtin_inff();
  const uint64_t best = block_max_u64(thread_argmax<kEpt2>(p, c.lo, c.hi), red);
  if (threadIdx.x == 0) a.smp_key[((int64_t)b * (a.K + 1) + r) * a.nch2 + ch] = best;
}

// grid B: the sampled tokens of each sequence -> its output.  Every
// sequence row's keys are loaded with the metadata, in one round trip.
__global__ __launch_bounds__(kThreads) void stoch_finalize_kernel(StochArgs a) {
  __shared__ uint64_t sKey[kMaxK + 1];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int K = a.K;
  if (tid <= K) sKey[tid] = 0;
  const int32_t* dec = a.dec + 4 * b;
  const int d0 = dec[0], d2 = dec[2], d3 = dec[3];
  const bool ngram = !has_rows(a, b);
  const int nd = K == 0 ? 0 : a.num_drafts[b];
  const int32_t dr = tid < K ? a.drafts[(int64_t)b * K + tid] : 0;
  const int32_t ac = tid <= K ? a.acc[(int64_t)b * (K + 1) + tid] : 0;
  const int total = (K + 1) * a.nch2;
  const uint64_t* keys = a.smp_key + (int64_t)b * (K + 1) * a.nch2;
  for (int e0 = 0; e0 < total; e0 += 8 * kThreads) {  // 8 loads in flight per thread
    uint64_t k[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + tid + u * kThreads;
      k[u] = e < total ? keys[e] : 0ull;
    }
    __syncthreads();  // sKey's zeros (and, first time round, every load above)
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + tid + u * kThreads;
      if (e < total) atomicMax((unsigned long long*)&sKey[e / a.nch2], (unsigned long long)k[u]);
    }
  }
  __syncthreads();
  if (d3 || tid >= 64) return;  // greedy sequence: finished by the accept walk
  const int lane = tid;
  int32_t* out = a.out_tokens + (int64_t)b * a.out_seq;
  if (!ngram) {
    if (lane < d2) out[lane] = ac;
    if (lane == d2) out[d2] = (int32_t)key_index(sKey[d0]);
    if (lane == 0) a.out_len[b] = d2 + 1;
    return;
  }
  // rejection_sampler.py:76-85: accept while the target sample equals the draft
  const int kb = min(max(nd, 0), K);
  const int32_t smp = lane <= kb ? (int32_t)key_index(sKey[lane]) : 0;
  const uint64_t miss = __ballot(lane < kb && smp != dr);
  const int n = miss ? __ffsll((long long)miss) - 1 : kb;
  if (lane <= n) out[lane] = smp;
  if (lane == 0) a.out_len[b] = n + 1;
}

// Chunks per row of the statistics pass and the slab width: 8192-element
// chunks (EPT 32) when the rows alone give the chip enough workgroups, else
// 2048-element chunks (EPT 8); at most kMaxChunks either way.
struct StatsPlan {
  int nch, ept;
};
StatsPlan stats_plan(int rows, int V) {
  StatsPlan p;
  const int wide = (V + kThreads * kEptWide - 1) / (kThreads * kEptWide);
  p.ept = (int64_t)rows * wide >= 1024 ? kEptWide : kEptNarrow;
  const int n = (V + kThreads * p.ept - 1) / (kThreads * p.ept);
  p.nch = n < 1 ? 1 : (n > kMaxChunks ? kMaxChunks : n);
  return p;
}
// the workspace is sized for the larger chunk count of the two widths
int max_stats_chunks(int V) {
  const int n = (V + kThreads * kEptNarrow - 1) / (kThreads * kEptNarrow);
  return n < 1 ? 1 : (n > kMaxChunks ? kMaxChunks : n);
}
int sample_chunks(int V) { return (V + kChunk2 - 1) / kChunk2; }

size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }

struct StochLayout {
  size_t st_max, st_sum, st_key, zpos, row_m, row_s, dec, acc, res_part, smp_key, total;
};

StochLayout stoch_layout(int B, int K, int nch, int nch2) {
  StochLayout L;
  const size_t R = 2 * (size_t)K + 1, K1 = (size_t)K + 1;
  size_t off = 0;
  L.st_max = off;   off += a256((size_t)B * R * nch * sizeof(float));
  L.st_sum = off;   off += a256((size_t)B * R * nch * sizeof(double));
  L.st_key = off;   off += a256((size_t)B * K1 * nch * sizeof(uint64_t));
  L.zpos = off;     off += a256((size_t)B * R * sizeof(float));
  L.row_m = off;    off += a256((size_t)B * R * sizeof(float));
  L.row_s = off;    off += a256((size_t)B * R * sizeof(double));
  L.dec = off;      off += a256((size_t)B * 4 * sizeof(int32_t));
  L.acc = off;      off += a256((size_t)B * K1 * sizeof(int32_t));
  L.res_part = off; off += a256((size_t)B * nch2 * 2 * sizeof(double));
  L.smp_key = off;  off += a256((size_t)B * K1 * nch2 * sizeof(uint64_t));
  L.total = off;
  return L;
}

bool bad_shape(int B, int K, int V, int dtype) {
  return B < 0 || K < 0 || K > kMaxK || V <= 0 || (dtype != NSV_F32 && dtype != NSV_BF16);
}

template <typename T>
void launch_stats(const StochArgs& a, int ept, dim3 grid, hipStream_t s) {
  if (ept == kEptWide) hipLaunchKernelGGL((stoch_stats_kernel<T, kEptWide>), grid, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((stoch_stats_kernel<T, kEptNarrow>), grid, dim3(kThreads), 0, s, a);
}

// Fill the workspace views of `a` and launch the stochastic kernels.
// sample_rows: K+1 when a sequence may sample every row (n-gram mode),
// 1 when every sequence has draft rows.
int launch_stoch(StochArgs& a, const StochLayout& L, char* ws, int ept, int sample_rows, int dtype, int ndtype,
                 hipStream_t s) {
  a.st_max = (float*)(ws + L.st_max);
  a.st_sum = (double*)(ws + L.st_sum);
  a.st_key = (uint64_t*)(ws + L.st_key);
  a.zpos = (float*)(ws + L.zpos);
  a.row_m = (float*)(ws + L.row_m);
  a.row_s = (double*)(ws + L.row_s);
  a.dec = (int32_t*)(ws + L.dec);
  a.acc = (int32_t*)(ws + L.acc);
  a.res_part = (double*)(ws + L.res_part);
  a.smp_key = (uint64_t*)(ws + L.smp_key);
  const int B = a.B;
  const dim3 g1(B * a.rows, a.nch), g2(B, a.nch2), g3(B, a.nch2, sample_rows);
  const bool bf = dtype == NSV_BF16;
  if (bf) launch_stats<uint16_t>(a, ept, g1, s);
  else launch_stats<float>(a, ept, g1, s);
  int rc = nsv_launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(stoch_decide_kernel, dim3(B), dim3(kThreads), 0, s, a);
  if ((rc = nsv_launch_status())) return rc;
  if (a.draft) {
    if (bf) hipLaunchKernelGGL(stoch_residual_kernel<uint16_t>, g2, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL(stoch_residual_kernel<float>, g2, dim3(kThreads), 0, s, a);
    if ((rc = nsv_launch_status())) return rc;
  }
  if (bf && ndtype == NSV_BF16) hipLaunchKernelGGL((stoch_sample_kernel<uint16_t, uint16_t>), g3, dim3(kThreads), 0, s, a);
  else if (bf) hipLaunchKernelGGL((stoch_sample_kernel<uint16_t, float>), g3, dim3(kThreads), 0, s, a);
  else hipLaunchKernelGGL((stoch_sample_kernel<float, float>), g3, dim3(kThreads), 0, s, a);
  if ((rc = nsv_launch_status())) return rc;
  hipLaunchKernelGGL(stoch_finalize_kernel, dim3(B), dim3(kThreads), 0, s, a);
  return nsv_launch_status();
}

}  // namespace

extern "C" {

size_t nsv_accept_workspace_size(int B, int K, int V, int dtype, int stochastic) {
  if (bad_shape(B, K, V, dtype)) return 0;
  if (!stochastic) return a256((size_t)B * (K + 1) * max_stats_chunks(V) * sizeof(uint64_t));
  return stoch_layout(B, K, max_stats_chunks(V), sample_chunks(V)).total;
}

int nsv_accept_greedy(const void* target_logits, int64_t seq_stride, const int32_t* drafts,
                      const int32_t* num_drafts, int B, int K, int V, int dtype, int32_t* out_tokens,
                      int32_t* out_len, void* workspace, size_t workspace_bytes, void* stream) {
  if (bad_shape(B, K, V, dtype) || seq_stride < K + 1) return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!target_logits || (!drafts && K > 0) || !num_drafts || !out_tokens || !out_len) return NSV_ERR_ARG;
  const size_t need = nsv_accept_workspace_size(B, K, V, dtype, 0);
  if (!workspace || workspace_bytes < need) return NSV_ERR_WORKSPACE;
  const StatsPlan sp = stats_plan(B * (K + 1), V);
  GreedyArgs a;
  a.logits = target_logits;
  a.seq_stride = seq_stride;
  a.drafts = drafts;
  a.num_drafts = num_drafts;
  a.B = B;
  a.K = K;
  a.V = V;
  a.nch = sp.nch;
  a.keys = (uint64_t*)workspace;
  a.out_tokens = out_tokens;
  a.out_len = out_len;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(B * (K + 1), a.nch);
  if (dtype == NSV_BF16) {
    if (sp.ept == kEptWide) hipLaunchKernelGGL((greedy_argmax_kernel<uint16_t, kEptWide>), grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((greedy_argmax_kernel<uint16_t, kEptNarrow>), grid, dim3(kThreads), 0, s, a);
  } else {
    if (sp.ept == kEptWide) hipLaunchKernelGGL((greedy_argmax_kernel<float, kEptWide>), grid, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((greedy_argmax_kernel<float, kEptNarrow>), grid, dim3(kThreads), 0, s, a);
  }
  int rc = nsv_launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(greedy_finalize_kernel, dim3(B), dim3(kThreads), 0, s, a);
  return nsv_launch_status();
}

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
  const StochLayout L = stoch_layout(B, K, max_stats_chunks(V), sample_chunks(V));
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
  a.rows = draft_logits ? 2 * K + 1 : K + 1;
  const StatsPlan sp = stats_plan(B * a.rows, V);
  a.nch = sp.nch;
  a.nch2 = sample_chunks(V);
  a.cdtype = dtype;
  a.out_tokens = out_tokens;
  a.out_seq = K + 1;
  a.out_len = out_len;
  const int sample_rows = (draft_logits && !draft_mode) ? 1 : K + 1;
  return launch_stoch(a, L, (char*)workspace, sp.ept, sample_rows, dtype, dtype, (hipStream_t)stream);
}

size_t nsv_sample_workspace_size(int B, int V, int dtype) {
  if (bad_shape(B, 0, V, dtype)) return 0;
  return stoch_layout(B, 0, max_stats_chunks(V), sample_chunks(V)).total + a256((size_t)B * sizeof(int32_t));
}

int nsv_sample(const void* logits, int64_t row_stride, const float* temperature, const float* noise, int B, int V,
               int dtype, int32_t* out_tokens, int64_t out_stride, void* workspace, size_t workspace_bytes,
               void* stream) {
  if (bad_shape(B, 0, V, dtype) || row_stride < V || row_stride % V || out_stride < 1) return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!logits || !temperature || !noise || !out_tokens) return NSV_ERR_ARG;
  const StochLayout L = stoch_layout(B, 0, max_stats_chunks(V), sample_chunks(V));
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
  a.rows = 1;
  const StatsPlan sp = stats_plan(B, V);
  a.nch = sp.nch;
  a.nch2 = sample_chunks(V);
  a.cdtype = NSV_F32;  // logits / (fp32 tensor) promotes to fp32 (layers/sampler.py:20-23)
  a.out_tokens = out_tokens;
  a.out_seq = out_stride;
  a.out_len = (int32_t*)((char*)workspace + L.total);
  return launch_stoch(a, L, (char*)workspace, sp.ept, 1, dtype, NSV_F32, (hipStream_t)stream);
}

}  // extern "C"
