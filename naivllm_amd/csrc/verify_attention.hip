// Paged multi-token verify attention and paged KV scatter for gfx950.
//
// Behaviour follows the reference's Triton path
// (src/myvllm/layers/attention.py:522-668 verify, :9-112 KV store); the
// decomposition is this library's own:
//
//   * one workgroup per (sequence, kv-head, key split).  The workgroup reads
//     each K/V byte of its split exactly once and serves every query row of
//     the GQA group from it (the reference re-reads K/V once per query head);
//   * the query rows of a GQA group are packed into the M dimension of a
//     16x16x32 bf16 MFMA: rows m = g * QL + t for group member g and
//     verify row t, padded to 16 * MT rows;
//   * S^T = K Q^T is computed so that the MFMA result layout is directly the
//     B operand of O^T = V^T P^T (no register shuffles between the two
//     products); V is staged through LDS once per 32-key tile and read back
//     transposed;
//   * splits of a long context produce fp32 partials (unnormalised O plus
//     log2-domain max and sum) that a second kernel merges; a sequence that
//     fits in one split is normalised and written directly.

#include "common.h"

namespace {

constexpr int kTile = 32;        // keys per wave iteration
constexpr int kWaves = 4;        // waves per workgroup (bf16 path)
constexpr float kNegInf = -__builtin_inff();

struct VerifyArgs {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_tables;
  const int64_t* context_lens;
  const int32_t* cu_seqlens_q;
  const int64_t* positions;
  void* out;
  float* part_o;   // [B, Hkv, S, Mv, D]  unnormalised split outputs
  float* part_ml;  // [B, Hkv, S, Mv, 2]  (running max, running sum), log2 domain
  float scale_log2;  // softmax scale * log2(e)
  int H, Hkv, G, bs_log2, max_blocks, QL, Mv, S, split_tokens;
};

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// Keys of sequence b the kernels visit: never past the block table's width,
// the bound the reference's chunk loop has (layers/attention.py:572).
__device__ __forceinline__ int context_len(const VerifyArgs& a, int b) {
  const int64_t ctx = a.context_lens[b];
  const int64_t cap = (int64_t)a.max_blocks << a.bs_log2;
  return (int)(ctx < 0 ? 0 : (ctx < cap ? ctx : cap));
}

// Number of key splits sequence b actually uses (>= 1 so that an empty
// sequence still gets its rows written).
__device__ __forceinline__ int splits_for(int ctx, int split_tokens) {
  return ctx <= split_tokens ? 1 : (ctx + split_tokens - 1) / split_tokens;
}

// ---------------------------------------------------------------------------
// bf16 path: 4 waves, MFMA 16x16x32.
// ---------------------------------------------------------------------------
template <int MT, int DH>
__global__ __launch_bounds__(256, 2) void verify_attn_bf16_kernel(VerifyArgs a) {
  constexpr int KS = DH / 32;           // k-steps of S^T = K Q^T
  constexpr int DT = DH / 16;           // 16-wide d tiles of O^T
  constexpr int MP = MT * 16;           // padded query rows
  constexpr int VSTR = DH + 4;          // staged V row stride (bf16); 8-byte aligned and
                                        // bank-conflict free for the transposed reads
  constexpr int VCH = DH / 8;           // 16-byte chunks per V row
  constexpr int VLOADS = kTile * VCH / NSV_WAVE;
  constexpr int OSTR = DH + 1;

  __shared__ __attribute__((aligned(16))) uint16_t v_lds[kWaves][kTile * VSTR];
  __shared__ float red_m[kWaves][MP];
  __shared__ float red_l[kWaves][MP];
  __shared__ float row_l[MP];
  __shared__ float row_ms[MP];
  __shared__ float red_o[MP * OSTR];

  const int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g4 = lane >> 4, c = lane & 15;

  const int ctx = context_len(a, b);
  const int nsplit = splits_for(ctx, a.split_tokens);
  if (split >= nsplit) return;  // uniform per workgroup
  const int tok_begin = split * a.split_tokens;
  const int tok_end = min(ctx, tok_begin + a.split_tokens);
  const int q0 = a.cu_seqlens_q[b];
  const int qlen = a.cu_seqlens_q[b + 1] - q0;

  // Q^T as the B operand: lane (g4, c) holds row m = 16*mt + c, dims 32*ks + 8*g4 .. +7.
  bf16x8 qB[MT][KS];
  int qpos[MT];
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + c;
    const int g = m / a.QL, t = m - g * a.QL;
    const bool ok = (m < a.Mv) && (t < qlen);
    int pos = -1;
    const bf16_t* qrow = nullptr;
    if (ok) {
      pos = (int)a.positions[q0 + t];
      qrow = (const bf16_t*)a.q + ((int64_t)(q0 + t) * a.H + hk * a.G + g) * DH;
    }
    qpos[mt] = pos;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qB[mt][ks] = as_bf16x8(ok ? load16(qrow + ks * 32 + g4 * 8) : zero4);
  }

  float m_run[MT], l_run[MT];
  f32x4 acc[DT][MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    m_run[mt] = kNegInf;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int32_t* bt = a.block_tables + (int64_t)b * a.max_blocks;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const int64_t tok_stride = (int64_t)a.Hkv * DH;
  const bf16_t* kbase = (const bf16_t*)a.k_cache + hk * DH;
  const bf16_t* vbase = (const bf16_t*)a.v_cache + hk * DH;
  uint16_t* vl = v_lds[w];

  const int ntiles = (tok_end - tok_begin + kTile - 1) / kTile;
  const int niter = (ntiles + kWaves - 1) / kWaves;  // same trip count in every wave

  for (int it = 0; it < niter; ++it) {
    const int n0 = tok_begin + (it * kWaves + w) * kTile;

    // Which of the tile's 32 keys exist (inside the split, page mapped).
    bool key_ok = false;
    if (lane < kTile) {
      const int n = n0 + lane;
      if (n < tok_end) key_ok = bt[n >> a.bs_log2] >= 0;
    }
    const uint64_t kmask = __ballot(key_ok);

    // K as the A operand: lane (g4, c) holds key 16*t + c, dims 32*ks + 8*g4 .. +7.
    u32x4 kraw[2][KS];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int nr = t * 16 + c;
      const bool ok = (kmask >> nr) & 1;
      const bf16_t* kp = nullptr;
      if (ok) {
        const int n = n0 + nr;
        kp = kbase + ((int64_t)bt[n >> a.bs_log2] * (bs_mask + 1) + (n & bs_mask)) * tok_stride;
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kraw[t][ks] = ok ? load16(kp + ks * 32 + g4 * 8) : zero4;
    }
    // V rows, coalesced: 64 lanes cover 64 * 16 bytes = 4 (DH=128) key rows per load.
    u32x4 vraw[VLOADS];
#pragma unroll
    for (int r = 0; r < VLOADS; ++r) {
      const int idx = r * NSV_WAVE + lane;
      const int tk = idx / VCH, dc = idx - tk * VCH;
      const bool ok = (kmask >> tk) & 1;
      vraw[r] = zero4;
      if (ok) {
        const int n = n0 + tk;
        vraw[r] = load16(vbase + ((int64_t)bt[n >> a.bs_log2] * (bs_mask + 1) + (n & bs_mask)) * tok_stride +
                         dc * 8);
      }
    }

    // S^T tile: lane (g4, c), element i -> key 16*t + 4*g4 + i, query row 16*mt + c.
    f32x4 sacc[2][MT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kraw[t][ks]), qB[mt][ks], s, 0, 0, 0);
        sacc[t][mt] = s;
      }

    // Online softmax in the log2 domain; every row's statistics are held
    // redundantly by the four lanes that share its column c.
    bf16x8 pB[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float x[2][4];
      float mx = kNegInf;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int nr = t * 16 + g4 * 4 + i;
          const bool ok = ((kmask >> nr) & 1) && (n0 + nr <= qpos[mt]);
          x[t][i] = ok ? sacc[t][mt][i] * a.scale_log2 : kNegInf;
          mx = fmaxf(mx, x[t][i]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, NSV_WAVE));
      mx = fmaxf(mx, __shfl_xor(mx, 32, NSV_WAVE));
      const float m_new = fmaxf(m_run[mt], mx);
      const float ms = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = exp2f(m_run[mt] - ms);
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = exp2f(x[t][i] - ms);
          x[t][i] = p;
          sum += p;
        }
      sum += __shfl_xor(sum, 16, NSV_WAVE);
      sum += __shfl_xor(sum, 32, NSV_WAVE);
      l_run[mt] = l_run[mt] * alpha + sum;
      m_run[mt] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt][mt] *= alpha;
      // P^T as the B operand of O^T = V^T P^T, rounded to bf16 like the
      // reference's `p.to(v.dtype)`.  Element j covers key kmap(g4, j).
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pB[mt][i] = (bf16_t)x[0][i];
        pB[mt][4 + i] = (bf16_t)x[1][i];
      }
    }

    // Stage V (this wave's private LDS slice; LDS ops of one wave complete in order).
#pragma unroll
    for (int r = 0; r < VLOADS; ++r) {
      const int idx = r * NSV_WAVE + lane;
      const int tk = idx / VCH, dc = idx - tk * VCH;
      uint2* dst = reinterpret_cast<uint2*>(vl + tk * VSTR + dc * 8);
      dst[0] = make_uint2(vraw[r].x, vraw[r].y);
      dst[1] = make_uint2(vraw[r].z, vraw[r].w);
    }
    __builtin_amdgcn_wave_barrier();

    // O^T += V^T P^T: lane (g4, c) reads V[kmap(g4, j)][16*dt + c] for j = 0..7,
    // kmap(g, j) = 4g + j (j < 4), 16 + 4g + (j - 4) (j >= 4) — the keys its S^T
    // elements hold, so the P operand needs no data movement.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint16_t* col = vl + dt * 16 + c;
      uint32_t v01 = (uint32_t)col[(g4 * 4 + 0) * VSTR] | ((uint32_t)col[(g4 * 4 + 1) * VSTR] << 16);
      uint32_t v23 = (uint32_t)col[(g4 * 4 + 2) * VSTR] | ((uint32_t)col[(g4 * 4 + 3) * VSTR] << 16);
      uint32_t v45 = (uint32_t)col[(16 + g4 * 4 + 0) * VSTR] | ((uint32_t)col[(16 + g4 * 4 + 1) * VSTR] << 16);
      uint32_t v67 = (uint32_t)col[(16 + g4 * 4 + 2) * VSTR] | ((uint32_t)col[(16 + g4 * 4 + 3) * VSTR] << 16);
      const bf16x8 vA = as_bf16x8(u32x4{v01, v23, v45, v67});
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[dt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vA, pB[mt], acc[dt][mt], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the four waves' (max, sum, O) ---------------------------------
  if (g4 == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      red_m[w][mt * 16 + c] = m_run[mt];
      red_l[w][mt * 16 + c] = l_run[mt];
    }
  }
  __syncthreads();
  if (tid < MP) {
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, red_m[ww][tid]);
    const float ms = (M == kNegInf) ? 0.f : M;
    float L = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) L += red_l[ww][tid] * exp2f(red_m[ww][tid] - ms);
    row_ms[tid] = M;
    row_l[tid] = L;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + c;
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, red_m[ww][m]);
    const float fac = exp2f(m_run[mt] - ((M == kNegInf) ? 0.f : M));
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt][mt] *= fac;
  }
  for (int ww = 0; ww < kWaves; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float* o = &red_o[(mt * 16 + c) * OSTR + dt * 16 + g4 * 4 + i];
            *o = (ww == 0 ? 0.f : *o) + acc[dt][mt][i];
          }
    }
    __syncthreads();
  }

  if (nsplit == 1) {
    bf16_t* out = (bf16_t*)a.out;
    for (int idx = tid; idx < a.Mv * DH; idx += 256) {
      const int m = idx / DH, d = idx - m * DH;
      const int g = m / a.QL, t = m - g * a.QL;
      if (t >= qlen) continue;
      const float L = row_l[m];
      const float v = L > 0.f ? red_o[m * OSTR + d] / L : 0.f;
      out[((int64_t)(q0 + t) * a.H + hk * a.G + g) * DH + d] = (bf16_t)v;
    }
  } else {
    const int64_t base = (((int64_t)b * a.Hkv + hk) * a.S + split) * a.Mv;
    for (int idx = tid; idx < a.Mv * DH; idx += 256) {
      const int m = idx / DH, d = idx - m * DH;
      a.part_o[(base + m) * DH + d] = red_o[m * OSTR + d];
    }
    if (tid < a.Mv) {
      a.part_ml[(base + tid) * 2 + 0] = row_ms[tid];
      a.part_ml[(base + tid) * 2 + 1] = row_l[tid];
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 path: one wave per workgroup, VALU dot products (exact fp32 math, the
// 1e-5 contract).  Lane = key for Q.K, lane = head dim for P.V.
// ---------------------------------------------------------------------------
template <int MT, int DH>
__global__ __launch_bounds__(64) void verify_attn_f32_kernel(VerifyArgs a) {
  constexpr int MP = MT * 16;
  constexpr int E = DH / 64;
  __shared__ __attribute__((aligned(16))) float q_s[MP][DH];
  __shared__ float p_s[MP][NSV_WAVE];
  __shared__ int pos_s[MP];

  const int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int ctx = context_len(a, b);
  const int nsplit = splits_for(ctx, a.split_tokens);
  if (split >= nsplit) return;
  const int tok_begin = split * a.split_tokens;
  const int tok_end = min(ctx, tok_begin + a.split_tokens);
  const int q0 = a.cu_seqlens_q[b];
  const int qlen = a.cu_seqlens_q[b + 1] - q0;

  for (int idx = lane; idx < MP * DH; idx += NSV_WAVE) {
    const int m = idx / DH, d = idx - m * DH;
    const int g = m / a.QL, t = m - g * a.QL;
    const bool ok = (m < a.Mv) && (t < qlen);
    q_s[m][d] = ok ? ((const float*)a.q)[((int64_t)(q0 + t) * a.H + hk * a.G + g) * DH + d] : 0.f;
  }
  if (lane < MP) {
    const int m = lane;
    const int g = m / a.QL, t = m - g * a.QL;
    const bool ok = (m < a.Mv) && (t < qlen);
    pos_s[m] = ok ? (int)a.positions[q0 + t] : -1;
  }
  __syncthreads();

  float m_run[MP], l_run[MP], acc[MP][E];
#pragma unroll
  for (int m = 0; m < MP; ++m) {
    m_run[m] = kNegInf;
    l_run[m] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[m][e] = 0.f;
  }

  const int32_t* bt = a.block_tables + (int64_t)b * a.max_blocks;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const int64_t tok_stride = (int64_t)a.Hkv * DH;
  const float* kbase = (const float*)a.k_cache + hk * DH;
  const float* vbase = (const float*)a.v_cache + hk * DH;

  for (int n0 = tok_begin; n0 < tok_end; n0 += NSV_WAVE) {
    const int n = n0 + lane;
    int blk = -1;
    if (n < tok_end) blk = bt[n >> a.bs_log2];
    const bool ok = blk >= 0;
    float s[MP];
#pragma unroll
    for (int m = 0; m < MP; ++m) s[m] = 0.f;
    if (ok) {
      const float* kp = kbase + ((int64_t)blk * (bs_mask + 1) + (n & bs_mask)) * tok_stride;
      for (int d = 0; d < DH; d += 4) {
        const float4 kv = *reinterpret_cast<const float4*>(kp + d);
#pragma unroll
        for (int m = 0; m < MP; ++m) {
          const float4 qv = *reinterpret_cast<const float4*>(&q_s[m][d]);
          s[m] = fmaf(qv.x, kv.x, s[m]);
          s[m] = fmaf(qv.y, kv.y, s[m]);
          s[m] = fmaf(qv.z, kv.z, s[m]);
          s[m] = fmaf(qv.w, kv.w, s[m]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MP; ++m) {
      const float x = (ok && n <= pos_s[m]) ? s[m] * a.scale_log2 : kNegInf;
      const float m_new = fmaxf(m_run[m], wave_max(x));
      const float ms = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = exp2f(m_run[m] - ms);
      const float p = exp2f(x - ms);
      l_run[m] = l_run[m] * alpha + wave_sum(p);
      m_run[m] = m_new;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[m][e] *= alpha;
      p_s[m][lane] = p;
    }
    __syncthreads();
    const int jn = min(NSV_WAVE, tok_end - n0);
    for (int j = 0; j < jn; ++j) {
      const int nn = n0 + j;
      const int bj = bt[nn >> a.bs_log2];
      if (bj < 0) continue;  // uniform across the wave
      const float* vp = vbase + ((int64_t)bj * (bs_mask + 1) + (nn & bs_mask)) * tok_stride;
      float v[E];
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = vp[lane + 64 * e];
#pragma unroll
      for (int m = 0; m < MP; ++m) {
        const float p = p_s[m][j];
#pragma unroll
        for (int e = 0; e < E; ++e) acc[m][e] = fmaf(p, v[e], acc[m][e]);
      }
    }
    __syncthreads();
  }

  if (nsplit == 1) {
    float* out = (float*)a.out;
#pragma unroll
    for (int m = 0; m < MP; ++m) {
      const int g = m / a.QL, t = m - g * a.QL;
      if (m >= a.Mv || t >= qlen) continue;
#pragma unroll
      for (int e = 0; e < E; ++e)
        out[((int64_t)(q0 + t) * a.H + hk * a.G + g) * DH + lane + 64 * e] =
            l_run[m] > 0.f ? acc[m][e] / l_run[m] : 0.f;
    }
  } else {
    const int64_t base = (((int64_t)b * a.Hkv + hk) * a.S + split) * a.Mv;
#pragma unroll
    for (int m = 0; m < MP; ++m) {
      if (m >= a.Mv) continue;
#pragma unroll
      for (int e = 0; e < E; ++e) a.part_o[(base + m) * DH + lane + 64 * e] = acc[m][e];
      if (lane == 0) {
        a.part_ml[(base + m) * 2 + 0] = m_run[m];
        a.part_ml[(base + m) * 2 + 1] = l_run[m];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Split merge: one workgroup per (row, kv-head, sequence), one lane per dim.
// ---------------------------------------------------------------------------
template <typename OutT>
__global__ __launch_bounds__(128) void verify_combine_kernel(VerifyArgs a, int DH) {
  const int m = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int d = threadIdx.x;
  const int ctx = context_len(a, b);
  const int nsplit = splits_for(ctx, a.split_tokens);
  if (nsplit <= 1) return;  // written by the attention kernel itself
  const int g = m / a.QL, t = m - g * a.QL;
  const int q0 = a.cu_seqlens_q[b];
  const int qlen = a.cu_seqlens_q[b + 1] - q0;
  if (t >= qlen || d >= DH) return;
  const int64_t base = (((int64_t)b * a.Hkv + hk) * a.S) * a.Mv + m;
  float M = kNegInf;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, a.part_ml[(base + (int64_t)s * a.Mv) * 2]);
  const float ms = (M == kNegInf) ? 0.f : M;
  float L = 0.f, o = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const int64_t r = base + (int64_t)s * a.Mv;
    const float f = exp2f(a.part_ml[r * 2] - ms);
    L += a.part_ml[r * 2 + 1] * f;
    o += a.part_o[r * DH + d] * f;
  }
  const float v = L > 0.f ? o / L : 0.f;
  ((OutT*)a.out)[((int64_t)(q0 + t) * a.H + hk * a.G + g) * DH + d] = (OutT)v;
}

// ---------------------------------------------------------------------------
// KV scatter: a cache row [Hkv, D] is contiguous in both the step's K/V and
// the paged cache, and its cache row index is the slot itself.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void store_kv_kernel(const u32x4* __restrict__ key, const u32x4* __restrict__ value,
                                                       u32x4* __restrict__ k_cache, u32x4* __restrict__ v_cache,
                                                       const int64_t* __restrict__ slots, int T, int chunks) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)T * chunks) return;
  const int t = (int)(idx / chunks), ch = (int)(idx - (int64_t)t * chunks);
  const int64_t slot = slots[t];
  if (slot < 0) return;
  k_cache[slot * chunks + ch] = key[(int64_t)t * chunks + ch];
  v_cache[slot * chunks + ch] = value[(int64_t)t * chunks + ch];
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct Plan {
  int G, QL, Mv, MT, split, S;
};

int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

int make_plan(int B, int H, int Hkv, int D, int block_size, int max_blocks, int max_q_len, int dtype,
              int kv_split_tokens, Plan* p) {
  if (B < 0 || H <= 0 || Hkv <= 0 || max_blocks <= 0 || max_q_len <= 0) return NSV_ERR_ARG;
  if (dtype != NSV_F32 && dtype != NSV_BF16) return NSV_ERR_ARG;
  if (H % Hkv) return NSV_ERR_UNSUPPORTED;
  if (D != 64 && D != 128) return NSV_ERR_UNSUPPORTED;
  if (ilog2_exact(block_size) < 0) return NSV_ERR_UNSUPPORTED;
  p->G = H / Hkv;
  p->QL = max_q_len;
  p->Mv = p->G * max_q_len;
  if (p->Mv > 64) return NSV_ERR_UNSUPPORTED;
  p->MT = (p->Mv + 15) / 16;
  const int64_t max_ctx = (int64_t)max_blocks * block_size;
  if (max_ctx > (int64_t)1 << 30) return NSV_ERR_UNSUPPORTED;
  int split = kv_split_tokens;
  if (split < 0 || (split % 128)) return NSV_ERR_ARG;
  if (split == 0) {
    // Enough workgroups to cover the chip a few times over, without
    // letting the fp32 partials grow past a few percent of the KV bytes.
    const int64_t target = dtype == NSV_BF16 ? 2048 : 1024;
    split = dtype == NSV_BF16 ? 128 : 256;
    while ((int64_t)B * Hkv * ((max_ctx + split - 1) / split) > target && split < 8192) split *= 2;
  }
  p->split = split;
  p->S = (int)((max_ctx + split - 1) / split);
  return NSV_OK;
}

size_t workspace_bytes_for(int B, int Hkv, int D, const Plan& p) {
  if (p.S <= 1) return 0;
  return (size_t)B * Hkv * p.S * p.Mv * (size_t)(D + 2) * sizeof(float);
}

template <int MT>
void launch_bf16(const VerifyArgs& a, int D, dim3 grid, hipStream_t s) {
  if (D == 128)
    hipLaunchKernelGGL((verify_attn_bf16_kernel<MT, 128>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((verify_attn_bf16_kernel<MT, 64>), grid, dim3(256), 0, s, a);
}

template <int MT>
void launch_f32(const VerifyArgs& a, int D, dim3 grid, hipStream_t s) {
  if (D == 128)
    hipLaunchKernelGGL((verify_attn_f32_kernel<MT, 128>), grid, dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL((verify_attn_f32_kernel<MT, 64>), grid, dim3(64), 0, s, a);
}

}  // namespace

extern "C" {

int nsv_version(void) { return 100; }

const char* nsv_error_string(int code) {
  switch (code) {
    case NSV_OK: return "ok";
    case NSV_ERR_ARG: return "invalid argument";
    case NSV_ERR_UNSUPPORTED: return "unsupported shape";
    case NSV_ERR_WORKSPACE: return "workspace missing or too small";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}

size_t nsv_verify_attention_workspace_size(int B, int H, int Hkv, int D, int block_size, int max_blocks,
                                           int max_q_len, int dtype, int kv_split_tokens) {
  Plan p;
  if (make_plan(B, H, Hkv, D, block_size, max_blocks, max_q_len, dtype, kv_split_tokens, &p) != NSV_OK) return 0;
  return workspace_bytes_for(B, Hkv, D, p);
}

int nsv_verify_attention(void* out, const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* block_tables, const int64_t* context_lens, const int32_t* cu_seqlens_q,
                         const int64_t* positions, float scale, int B, int T, int H, int Hkv, int D, int block_size,
                         int max_blocks, int max_q_len, int dtype, int kv_split_tokens, void* workspace,
                         size_t workspace_bytes, void* stream) {
  Plan p;
  int rc = make_plan(B, H, Hkv, D, block_size, max_blocks, max_q_len, dtype, kv_split_tokens, &p);
  if (rc != NSV_OK) return rc;
  if (T < 0) return NSV_ERR_ARG;
  if (B == 0 || T == 0) return NSV_OK;
  if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens || !cu_seqlens_q || !positions)
    return NSV_ERR_ARG;
  const size_t need = workspace_bytes_for(B, Hkv, D, p);
  if (need && (!workspace || workspace_bytes < need)) return NSV_ERR_WORKSPACE;

  VerifyArgs a;
  a.q = q;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.block_tables = block_tables;
  a.context_lens = context_lens;
  a.cu_seqlens_q = cu_seqlens_q;
  a.positions = positions;
  a.out = out;
  a.part_o = need ? (float*)workspace : nullptr;
  a.part_ml = need ? (float*)workspace + (size_t)B * Hkv * p.S * p.Mv * D : nullptr;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.H = H;
  a.Hkv = Hkv;
  a.G = p.G;
  a.bs_log2 = ilog2_exact(block_size);
  a.max_blocks = max_blocks;
  a.QL = p.QL;
  a.Mv = p.Mv;
  a.S = p.S;
  a.split_tokens = p.split;

  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(p.S, Hkv, B);
  if (dtype == NSV_BF16) {
    switch (p.MT) {
      case 1: launch_bf16<1>(a, D, grid, s); break;
      case 2: launch_bf16<2>(a, D, grid, s); break;
      case 3: launch_bf16<3>(a, D, grid, s); break;
      default: launch_bf16<4>(a, D, grid, s); break;
    }
  } else {
    switch (p.MT) {
      case 1: launch_f32<1>(a, D, grid, s); break;
      case 2: launch_f32<2>(a, D, grid, s); break;
      case 3: launch_f32<3>(a, D, grid, s); break;
      default: launch_f32<4>(a, D, grid, s); break;
    }
  }
  rc = nsv_launch_status();
  if (rc != NSV_OK || p.S <= 1) return rc;
  const dim3 cgrid(p.Mv, Hkv, B);
  if (dtype == NSV_BF16)
    hipLaunchKernelGGL(verify_combine_kernel<bf16_t>, cgrid, dim3(128), 0, s, a, D);
  else
    hipLaunchKernelGGL(verify_combine_kernel<float>, cgrid, dim3(128), 0, s, a, D);
  return nsv_launch_status();
}

int nsv_store_kv(const void* key, const void* value, void* k_cache, void* v_cache, const int64_t* slot_mapping,
                 int T, int Hkv, int D, int block_size, int dtype, void* stream) {
  if (T < 0 || Hkv <= 0 || D <= 0 || block_size <= 0) return NSV_ERR_ARG;
  if (dtype != NSV_F32 && dtype != NSV_BF16) return NSV_ERR_ARG;
  if (T == 0) return NSV_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return NSV_ERR_ARG;
  const int elt = dtype == NSV_BF16 ? 2 : 4;
  const int64_t row_bytes = (int64_t)Hkv * D * elt;
  if (row_bytes % 16) return NSV_ERR_UNSUPPORTED;
  const int chunks = (int)(row_bytes / 16);
  const int64_t total = (int64_t)T * chunks;
  const int blocks = (int)((total + 255) / 256);
  hipLaunchKernelGGL(store_kv_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const u32x4*)key,
                     (const u32x4*)value, (u32x4*)k_cache, (u32x4*)v_cache, slot_mapping, T, chunks);
  return nsv_launch_status();
}

}  // extern "C"
