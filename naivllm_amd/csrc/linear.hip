// Few-row linear layers of the Qwen3 verify forward for gfx950 (bf16 in,
// fp32 accumulation, one bf16 rounding per output).
//
// The verify forward multiplies B*(K+1) activation rows (72 at batch 8) by weight
// matrices of 2-300 MB, so streaming the weights, not arithmetic, bounds
// every projection.  A workgroup owns 16 output columns (16 weight rows):
// its 8 waves take 32- to 128-element chunks of the reduction dimension in
// turn, load their slice of the 16 rows and of every activation row as
// whole-row 16-byte loads (4 or 8 lanes cover one row's contiguous chunk),
// reshape both through a per-wave
// LDS tile into the MFMA operand layout and multiply them
// (v_mfma_f32_16x16x32_bf16, rows padded to 16; more than 80 rows take
// further workgroup rows of the grid); the waves' partial
// products are summed through LDS.  The next chunk's loads are issued
// before the current chunk is multiplied.
//
// Fused stages (each removes a kernel launch and an activation round trip):
//   * prologue RMSNorm (norm_w != NULL): the activation is rmsnorm(r) *
//     norm_w with r the bf16 residual stream, computed as
//     inv(r) * (r W'^T), W' = bf16(W * norm_w) formed as the weight rows are
//     staged; sum(r^2) per row arrives as per-tile partial sums from the
//     producing linear and is added in a fixed order;
//   * epilogue SwiGLU: the weight is [gate; up] ([2I, K]); a tile takes 8
//     gate rows and the matching 8 up rows and writes silu(gate) * up;
//   * epilogue residual: r = bf16(x) + r (x the product) rewrites the
//     residual stream, and each tile writes its partial sum(r^2) per row
//     for the consumer's RMSNorm.
// Reference: layers/linear.py (the projections are F.linear),
// layers/layernorm.py:18-35 (residual RMSNorm), layers/activation.py:17-19
// (SiluAndMul), models/qwen3.py:129-151 and 197-227 (where they meet).

#include "common.h"

namespace {

constexpr int kLinWaves = 8;
constexpr int kLinThreads = kLinWaves * 64;
constexpr int kBN = 16;            // output columns per workgroup
constexpr int kMaxRows = 80;       // activation rows (5 MFMA row tiles)
// Arrival counters of split tiles: one fixed 64 KiB area at the front of
// the workspace, so calls of every shape find their counters at the same
// place, zero.  Tiles 0..255 each get their own 256-byte line (device-scope
// atomics on one line serialise, ~20 ns apiece); tile t + 256 k shares
// t's line.  Splitting needs fewer than 128 column tiles, well inside.
constexpr int kMaxCounterTiles = 16384;
constexpr int kMaxSplits = 4;      // workgroups a tile's reduction is split over, at most
__device__ __forceinline__ int lin_counter_slot(int tile) { return ((tile & 255) << 6) | (tile >> 8); }

struct LinearArgs {
  const uint16_t* x;       // [M, K]: activations, or the residual stream r (RMSNorm prologue)
  const uint16_t* norm_w;  // [K] RMSNorm weight, or null
  const float* ss_in;      // [nss_in, M] partial sums of r^2 (RMSNorm prologue)
  int nss_in;
  float eps;
  const uint16_t* w;       // [N, K]
  uint16_t* y;             // [M, N] (plain) or [M, N/2] (SwiGLU)
  uint16_t* resid;         // [M, N] residual stream, read and rewritten (residual epilogue)
  float* ss_out;           // [N/16, M] partial sums of r^2 (residual epilogue)
  int M, N, K;
  int ks;                  // workgroups per 16-column tile, each taking a share of the reduction
  float* part;             // [N/16, ks, 80, 16] their partial products (ks > 1)
  unsigned* counters;      // tile t's workgroups done so far at lin_counter_slot(t); every call leaves them zero
};

__device__ __forceinline__ bf16x8 to_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bfv(uint32_t word, int hi) { return __uint_as_float(hi ? (word & 0xffff0000u) : (word << 16)); }

// Chunk size and occupancy.  A grid of more workgroups than CUs (384 for
// gate_up) needs two resident per CU, or its last third starts only when
// the first workgroups end.  Measured on MI355X, two 8-wave workgroups share
// a CU at <= 64 KB of LDS each (61 KB did, 70 KB did not) and <= 128 VGPRs
// per lane: the small chunk (64 elements up to 32 rows, 32 beyond) keeps the
// per-wave staging of [16 + MP rows][KC] within that.  A grid that fits the
// CUs takes twice the chunk (half the round trips of a long reduction).
// (4-column tiles at 9 rows with 256-element chunks, every 2048-element
// reduction one chunk per wave issued at once: 5.80 us per o_proj/down call
// against 5.29 with 128.)
constexpr int lin_kc(int MT, bool small) { return (MT <= 2 ? 128 : 64) / (small ? 2 : 1); }

// Minimum waves per SIMD the compiler must allow (HIP's second
// __launch_bounds__ argument is amdgpu_waves_per_eu, not workgroups per
// CU): two resident 8-wave workgroups are 4 waves per SIMD, i.e. at most
// 128 VGPRs.  The 32-column SwiGLU tiles with half chunks need 150 VGPRs
// from two row tiles on (224+ with full chunks); bounded to 128 they spill,
// so they run one workgroup per CU and keep the half chunk for its shorter
// staging round trips (8B gate_up at 18 rows: 48.1 us, against 50.3 with
// full chunks and 52.5 with 16-column tiles).
constexpr int lin_waves_per_eu(int MT, bool small, int bnv) { return small && !(bnv == 32 && MT >= 2) ? 4 : 1; }

// BNV: output columns per workgroup, 16, or 8 (the upper 8 MFMA columns
// zero) where few rows and few tiles leave most CUs idle: half the weight
// rows per CU and twice the workgroups (o_proj and down at 9 rows: 64 -> 128
// workgroups, 4.9 -> 4.5 and 5.6 -> 5.0 us alone; at 18 rows 0.2 us each),
// or 32 (two 16-column MFMA tiles per wave) for wide SwiGLU projections.
template <int MT, bool NORM, int EPI, bool SMALL, int BNV = kBN>  // EPI 0: plain, 1: SwiGLU, 2: residual
__global__ __launch_bounds__(kLinThreads, lin_waves_per_eu(MT, SMALL, BNV)) void linear_kernel(LinearArgs a) {
  static_assert(BNV == kBN || (BNV == 8 && EPI != 1) || (BNV == 4 && EPI != 1 && !NORM && !SMALL) ||
                    (BNV == 32 && EPI == 1),
                "4- and 8-column tiles: plain and residual epilogues; 32-column tiles: SwiGLU");
  constexpr int MP = MT * 16;
  constexpr int WR = BNV > kBN ? BNV : kBN;  // staged weight rows (MFMA columns), BNV rounded up to 16
  constexpr int NTL = WR / 16;               // 16-column MFMA tiles per workgroup
  constexpr int KC = lin_kc(MT, SMALL);   // reduction elements per wave chunk
  constexpr int LPR = KC / 8;             // lanes per row of a whole-row load (16 bytes each)
  constexpr int RPI = 64 / LPR;           // rows per load instruction
  constexpr int STR = KC + 8;             // staged row stride (bf16): 16-byte reads of 16 rows hit distinct banks
  constexpr int WL = BNV / RPI;           // weight loads per lane and chunk (rows < BNV)
  constexpr int AL = MP / RPI;            // activation loads per lane and chunk
  constexpr int STAGE = kLinWaves * (WR + MP) * STR * 2;  // staged chunks, bytes
  constexpr int RED = kLinWaves * MP * (WR + 1) * 4;      // cross-wave partial products, bytes
  constexpr int SMEM = STAGE > RED ? STAGE : RED;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  __shared__ float inv_s[MP];
  __shared__ float ss_s[kLinThreads];

  // every argument in one batch: the empty statement uses them all, so the
  // compiler cannot defer one's load past the first use of another (each
  // deferred load is a dependent round trip before the first weight load)
  __asm__ volatile("" ::"s"(a.x), "s"(a.norm_w), "s"(a.ss_in), "s"(a.nss_in), "s"(a.eps), "s"(a.w), "s"(a.y),
                   "s"(a.resid), "s"(a.ss_out), "s"(a.M), "s"(a.N), "s"(a.K), "s"(a.ks), "s"(a.part), "s"(a.counters));
  const int tile = blockIdx.x;
  const int kz = blockIdx.z;  // this workgroup's share of the reduction (split-K)
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, c = lane & 15;
  const int rr = lane / LPR, cc = lane % LPR;  // whole-row load: row rr + RPI j, elements 8 cc .. 8 cc + 7
  const int K = a.K;
  // rows of this workgroup: chunk blockIdx.y of kMaxRows rows
  const int row0 = blockIdx.y * kMaxRows;
  const int M = min(a.M - row0, kMaxRows);

  // weight row of tile column col
  const int half = a.N >> 1;
  auto wrow = [&](int col) -> int64_t {
    constexpr int GC = BNV / 2;  // SwiGLU: gate rows, then the matching up rows
    if constexpr (EPI == 1) return col < GC ? tile * GC + col : half + tile * GC + (col - GC);
    else return (int64_t)tile * BNV + col;
  };
  // the reduction in chunks of KC elements, dealt round-robin to the
  // ks * 8 waves of the tile (worker u = 8 kz + w takes chunks u, u + 8 ks,
  // ...); a last partial chunk reads zeros past K
  const int nck = (K + KC - 1) / KC;
  const int worker = kz * kLinWaves + w, nworkers = a.ks * kLinWaves;
  const int nchunk = worker < nck ? (nck - worker + nworkers - 1) / nworkers : 0;
  const uint16_t* wp[WL];
#pragma unroll
  for (int j = 0; j < WL; ++j) wp[j] = a.w + wrow(rr + RPI * j) * K + cc * 8;
  // Activation rows through a buffer resource of exactly this chunk's M
  // rows: the loads of padding rows (rr + RPI j >= M) lie past its range
  // and return zeros without a memory access (they were clamped reads of
  // row M - 1 before; the staging zeroes those rows either way).  Every
  // load is still issued, so the compiler's wait counts stay exact.  Four
  // projections of a layer: 35.5 -> 35.1 us at 72 rows, 27.8 -> 27.6 at 36,
  // unchanged at 9 and 18; b8 round 1.521 -> 1.516 ms.
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x + (int64_t)row0 * K), (short)0, M * K * 2, 0x00020000);
  int xo[AL];  // byte offset of row rr + RPI j, elements 8 cc ..
#pragma unroll
  for (int j = 0; j < AL; ++j) xo[j] = ((rr + RPI * j) * K + cc * 8) * 2;

  struct Chunk {
    u32x4 wv[WL];  // weight rows rr + RPI j
    u32x4 xv[AL];  // activation rows rr + RPI j
    u32x4 nv;      // RMSNorm weight
    int k0;
    bool in;       // this lane's 8 elements lie inside the reduction
  };
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  // Every issue has the same loads, unconditionally (lanes past K read
  // elements 0.. and their values are replaced by zeros when staged): loads
  // under a branch leave the compiler unable to count them, and it then
  // waits for every load in flight, the next chunk's included, before a
  // chunk is multiplied.
  auto issue = [&](Chunk& ch, int k0) {
    ch.in = k0 + KC <= K || k0 + cc * 8 < K;
    const int kk = ch.in ? k0 : -cc * 8;
#pragma unroll
    for (int j = 0; j < WL; ++j) ch.wv[j] = load16_stream(wp[j] + kk);
#pragma unroll
    for (int j = 0; j < AL; ++j)
      ch.xv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[j] + kk * 2, 0, 0));
    if constexpr (NORM) ch.nv = *reinterpret_cast<const u32x4*>(a.norm_w + kk + cc * 8);
    ch.k0 = k0;
  };

  uint16_t* st = reinterpret_cast<uint16_t*>(smem) + w * (WR + MP) * STR;  // [WR weight + MP activation rows][STR]
  f32x4 acc[NTL][MT];
#pragma unroll
  for (int nt = 0; nt < NTL; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Chunk& ch) {
    // stage the chunk's rows (this wave's LDS rows; a wave's LDS ops complete
    // in order).  RMSNorm prologue: the weight rows take the norm weight,
    // W'[n][k] = bf16(W[n][k] * norm_w[k]), and 1 / rms scales each output
    // row at the end -- h W^T = inv * (r W'^T) -- which touches 16 rows per
    // chunk instead of every activation row.
#pragma unroll
    for (int j = 0; j < WL; ++j) {
      u32x4 v = ch.in ? ch.wv[j] : zero4;
      if constexpr (NORM) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[q] = pack_bf16x2(bfv(v[q], 0) * bfv(ch.nv[q], 0), bfv(v[q], 1) * bfv(ch.nv[q], 1));
      }
      *reinterpret_cast<u32x4*>(st + (rr + RPI * j) * STR + cc * 8) = v;
    }
#pragma unroll
    for (int j = 0; j < AL; ++j) {
      const int m = rr + RPI * j;
      *reinterpret_cast<u32x4*>(st + (WR + m) * STR + cc * 8) = m < M && ch.in ? ch.xv[j] : zero4;
    }
    __builtin_amdgcn_wave_barrier();
    // operand reads: lane (g4, c) takes row c, elements 32 s + 8 g4 .. +7
#pragma unroll
    for (int s = 0; s < KC / 32; ++s) {
      u32x4 bw[NTL];
#pragma unroll
      for (int nt = 0; nt < NTL; ++nt)
        bw[nt] = *reinterpret_cast<const u32x4*>(st + (nt * 16 + c) * STR + 32 * s + 8 * g4);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4 av = *reinterpret_cast<const u32x4*>(st + (WR + mt * 16 + c) * STR + 32 * s + 8 * g4);
#pragma unroll
        for (int nt = 0; nt < NTL; ++nt)
          acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(to_bf16x8(av), to_bf16x8(bw[nt]), acc[nt][mt], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- loads, in the order they are consumed: the residual elements of the
  // residual epilogue (they do not depend on the product: loaded now rather
  // than after the reduction, one memory round trip less at the end; the
  // tile's columns are read and rewritten by this workgroup only), the
  // producer's partial sums of squares of the RMSNorm prologue, then the
  // first two chunks of the two-stage pipeline, which stream in during the
  // prologue.  A wait for a load then never waits for a later one.
  uint2 resid_pre = make_uint2(0u, 0u);
  if constexpr (EPI == 2) {
    constexpr int QPR = BNV / 4;
    const int m = min(tid / QPR, M - 1), q = tid % QPR;  // threads past the tile's rows load one and leave it unused
    resid_pre = *reinterpret_cast<const uint2*>(a.resid + (int64_t)(row0 + m) * a.N + (int64_t)tile * BNV + 4 * q);
  }
  // RMSNorm prologue: 1 / rms per row from the producer's partial sums,
  // added in a fixed order (thread part p sums slots p, p + P, ...; row m
  // then sums the P part sums in order)
  constexpr int P = kLinThreads / MP;
  float ssv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int ssm = tid % MP, ssp = tid / MP;
  const bool ss_on = NORM && ssp < P && ssm < M;
  if constexpr (NORM) {
    // (unconditional loads, clamped to the last slot and row, zeros selected
    // afterwards, in the prologue: a load under a branch, or a value used
    // at once, is waited for on the spot)
    const float* src = a.ss_in + row0 + min(ssm, M - 1);
#pragma unroll
    for (int u = 0; u < 8; ++u) ssv[u] = src[(int64_t)min(ssp + u * P, a.nss_in - 1) * a.M];
  }
  Chunk A, B;
  // chunk i of this wave (past its last chunk: elements outside the
  // reduction, read and never multiplied)
  auto k_of = [&](int i) { return (worker + i * nworkers) * KC; };
  auto prologue = [&]() {
    if constexpr (BNV < kBN)  // weight rows BNV..15 are never loaded: zero once (after the first loads' issue)
      for (int i = lane; i < (kBN - BNV) * STR / 8; i += NSV_WAVE)
        reinterpret_cast<u32x4*>(st + BNV * STR)[i] = u32x4{0u, 0u, 0u, 0u};
    if constexpr (NORM) {
      // (the partial sums are taken here, after the chunks' loads were
      // issued: the empty statement keeps the compiler from adding them up,
      // and so waiting for them, ahead of those loads)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 8; ++u) __asm__ volatile("" : "+v"(ssv[u]) : : "memory");
      float s = 0.f;
      if (ss_on) {
#pragma unroll
        for (int u = 0; u < 8; ++u) s += ssp + u * P < a.nss_in ? ssv[u] : 0.f;
        const float* src = a.ss_in + row0 + ssm;
        for (int j0 = ssp + 8 * P; j0 < a.nss_in; j0 += 8 * P) {  // more slots: 8 loads in flight per round trip
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v[u] = j0 + u * P < a.nss_in ? src[(int64_t)(j0 + u * P) * a.M] : 0.f;
#pragma unroll
          for (int u = 0; u < 8; ++u) s += v[u];
        }
      }
      ss_s[tid] = s;
      lds_barrier();
      if (tid < MP) {
        float t = 0.f;
        for (int q = 0; q < P; ++q) t += ss_s[q * MP + tid];
        inv_s[tid] = rsqrtf(t / (float)K + a.eps);
      }
      lds_barrier();
    }
  };

  if (nchunk <= 1) {
    // (one chunk or none, the common case of a short reduction: no second
    // chunk's loads; the branch is uniform per wave, each side issues its
    // loads unconditionally so the prologue waits for the partial sums only,
    // and both run the prologue's barriers once)
    issue(A, k_of(0));
    prologue();
    if (nchunk == 1) compute(A);
  } else {
    issue(A, k_of(0));
    issue(B, k_of(1));
    prologue();
    // (a symmetric loop body that issues only chunks of this wave, no exit in
    // its middle, and each issue kept after the multiply that frees its
    // registers: the compiler then counts the loads in flight exactly, a
    // multiply waits for its own chunk only, and nothing is left in flight
    // past the last chunk; the last two or three chunks are peeled)
    int i = 0;
    for (; i + 3 < nchunk; i += 2) {
      compute(A);
      __builtin_amdgcn_sched_barrier(0);
      issue(A, k_of(i + 2));
      __builtin_amdgcn_sched_barrier(0);
      compute(B);
      __builtin_amdgcn_sched_barrier(0);
      issue(B, k_of(i + 3));
      __builtin_amdgcn_sched_barrier(0);
    }
    if (i + 2 < nchunk) {
      compute(A);
      __builtin_amdgcn_sched_barrier(0);
      issue(A, k_of(i + 2));
      __builtin_amdgcn_sched_barrier(0);
      compute(B);
      compute(A);
    } else {
      compute(A);
      compute(B);
    }
  }

  // ---- sum the waves' partial products: lane (g4, c) holds C[16mt + 4g4 + i][c]
  lds_barrier();  // every wave is done with its staged weights (red aliases them)
  float* red = reinterpret_cast<float*>(smem);  // [kLinWaves][MP][WR + 1]
#pragma unroll
  for (int nt = 0; nt < NTL; ++nt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(w * MP + mt * 16 + g4 * 4 + i) * (WR + 1) + nt * 16 + c] = acc[nt][mt][i];
  lds_barrier();
  // split reductions run on 16-column tiles only; after one, red's wave-0
  // slot holds the tile's total and the epilogue reads only that slot
  bool split_total = false;
  if (WR == kBN && a.ks > 1) {
    // ---- split-K: publish this workgroup's tile partial; the tile's last
    // workgroup to finish sums the ks partials in split order (deterministic)
    // and runs the epilogue.  Ordering without release/acquire (which on
    // gfx950 would write back and invalidate whole L2s): every partial is
    // written and read with the agent-scope cache policy (sc1: performed at
    // the device's point of coherence, never served from a stale cached
    // copy); each thread waits for its stores' acknowledgement (vmcnt(0))
    // before the barrier that precedes the arrival atomic, and the last
    // workgroup issues its loads only after the counter's value came back.
    const int m = tid >> 2, q = tid & 3;
    const bool item = tid < MP * 4 && m < M;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (item) {
      float w8[kLinWaves][4];  // every wave's sums first (one LDS round trip), then the adds
#pragma unroll
      for (int ww = 0; ww < kLinWaves; ++ww)
#pragma unroll
        for (int e = 0; e < 4; ++e) w8[ww][e] = red[(ww * MP + m) * (kBN + 1) + 4 * q + e];
#pragma unroll
      for (int ww = 0; ww < kLinWaves; ++ww)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += w8[ww][e];
    }
    const __amdgpu_buffer_rsrc_t prs = block_rsrc(a.part + (int64_t)tile * a.ks * (kMaxRows * kBN));
    // the item in one split's block (threads past the tile's items load item 0: their loads stay inside
    // the block, which ends 80 rows x 16 columns after its start)
    const unsigned ioff = item ? (unsigned)(m * kBN + 4 * q) * 4u : 0u;
    constexpr unsigned kSplitBytes = kMaxRows * kBN * 4u;                  // one split's block
    if (item) store16_agent(prs, ioff + (unsigned)kz * kSplitBytes, v);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    __shared__ int last;
    if (tid == 0)
      last = __hip_atomic_fetch_add(&a.counters[lin_counter_slot(tile)], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (unsigned)(a.ks - 1);
    __syncthreads();
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    if (tid == 0) __hip_atomic_store(&a.counters[lin_counter_slot(tile)], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // every other split's partial in one round trip (splits past ks and this
    // workgroup's own read its own block and are not used), then the sum in
    // split order, this workgroup's own partial from registers
    f32x4 pz[kMaxSplits];
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z) {
      const int zz = __builtin_amdgcn_readfirstlane(z < a.ks && z != kz ? z : kz);
      pz[z] = load16_agent(prs, ioff, (unsigned)zz * kSplitBytes);
    }
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z)
      if (z < a.ks) t += z == kz ? v : pz[z];
    if (item) {
#pragma unroll
      for (int e = 0; e < 4; ++e) red[m * (kBN + 1) + 4 * q + e] = t[e];
    }
    lds_barrier();
    split_total = true;
  }
  auto colsum = [&](int m, int col) {
    float v = red[m * (WR + 1) + col];
    if (!split_total) {
#pragma unroll
      for (int ww = 1; ww < kLinWaves; ++ww) v += red[(ww * MP + m) * (WR + 1) + col];
    }
    return NORM ? v * inv_s[m] : v;
  };
  if constexpr (EPI == 1) {
    // item = (row, 4 gate columns): silu(gate) * up for 4 outputs
    constexpr int GC = BNV / 2, QG = GC / 4;  // gate columns, items per row
    if (tid < MP * QG) {
      const int m = tid / QG, q = tid % QG;
      if (m < M) {
        uint32_t o[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float r2[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int col = 4 * q + 2 * j + e;
            const float g = bf16_bits_to_f32(f32_to_bf16_bits(colsum(m, col)));
            const float u = bf16_bits_to_f32(f32_to_bf16_bits(colsum(m, GC + col)));
            r2[e] = g / (1.f + __expf(-g)) * u;
          }
          o[j] = (uint32_t)f32_to_bf16_bits(r2[0]) | ((uint32_t)f32_to_bf16_bits(r2[1]) << 16);
        }
        *reinterpret_cast<uint2*>(a.y + (int64_t)(row0 + m) * half + tile * GC + 4 * q) = make_uint2(o[0], o[1]);
      }
    }
  } else {
    // item = (row, 4 columns)
    constexpr int QPR = BNV / 4;  // items per row
    const int m = tid / QPR, q = tid % QPR;
    float ss = 0.f;
    if (tid < MP * QPR && m < M) {
      const int64_t off = (int64_t)(row0 + m) * a.N + (int64_t)tile * BNV + 4 * q;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = bf16_bits_to_f32(f32_to_bf16_bits(colsum(m, 4 * q + e)));
      uint16_t* dst = EPI == 2 ? a.resid : a.y;
      if constexpr (EPI == 2) {
        const uint32_t rw[2] = {resid_pre.x, resid_pre.y};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = bf16_bits_to_f32(f32_to_bf16_bits(v[e] + bfv(rw[e >> 1], e & 1)));  // the residual stream is bf16
          ss = fmaf(v[e], v[e], ss);
        }
      }
      *reinterpret_cast<uint2*>(dst + off) =
          make_uint2((uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16),
                     (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16));
    }
    if constexpr (EPI == 2) {
      // the QPR threads of a row are adjacent lanes of one wave: fixed-order butterfly
      if constexpr (QPR >= 2) ss += __shfl_xor(ss, 1, NSV_WAVE);
      if constexpr (QPR == 4) ss += __shfl_xor(ss, 2, NSV_WAVE);
      if (tid < MP * QPR && m < M && q == 0) a.ss_out[(int64_t)tile * a.M + row0 + m] = ss;
    }
  }
}

// Compute units of the current device (256 on MI355X), queried once per
// device; a failed query assumes 256.
int lin_device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
      (void)hipGetLastError();
      cus = 256;
    }
    cached[dev] = cus;
  }
  return cached[dev];
}

// 8-column tiles: plain or residual epilogue without the RMSNorm prologue,
// at most 31 rows, fewer than 128 16-column tiles (no split reduction then).
bool linear_half_tiles(int M, int N, bool norm, int epi) {
  return !norm && epi != 1 && M <= 31 && N / kBN < 128 && N % 8 == 0;
}

// 4-column tiles where even 8-column tiles leave CUs idle and 4-column ones
// still fit one workgroup per CU (full chunks, no split reduction; the MFMA
// tile's other 12 weight rows stay zero).  Measured on MI355X (Qwen3-0.6B
// o_proj and down, N = 1024, in the replayed verify round): 5.73 -> 5.29 us
// per call at 9 rows (128 -> 256 workgroups), 6.80 -> 6.48 at 18.
bool linear_quarter_tiles(int M, int N, bool norm, int epi, int cus) {
  return linear_half_tiles(M, N, norm, epi) && N % 4 == 0 && N / 8 < cus && N / 4 <= cus;
}

// 32-column tiles (16 gate + 16 up rows) for the SwiGLU epilogue where the
// 16-column grid would need two workgroups per CU: each wave multiplies
// every staged activation chunk into two weight tiles, so a CU ingests
// fewer activation bytes per output column.  A wide grid that fits the CUs
// keeps the full chunk (one workgroup per CU, whole 128-byte rows at 33-80
// rows); a larger one takes half chunks up to 32 rows (two workgroups per
// CU at up to 16 rows, one beyond: see lin_waves_per_eu).  Measured on
// MI355X (gate_up alone, graph-replayed, rotating weights; 16-column tiles
// -> 32-column): 0.6B (6144 x 1024, 192 workgroups) 7.41 -> 6.84 us at 9
// rows, 11.26 -> 10.13 us at 72; 8B (24576 x 4096, 768 workgroups) 44.3 ->
// 38.3 us at 9 rows and 52.5 -> 48.1 at 18 (full chunks: 45.3 and 50.3),
// 76.1 -> 56.2 at 36 and 107.8 -> 69.3 at 72 (full chunks; half chunks:
// 57.6 and 81.4).  Only grids of >= 128 16-column tiles take them, where
// the reduction is never split (linear_splits), whatever the CU count.
bool linear_wide_tiles(int N, int epi, int cus) {
  return epi == 1 && N % 32 == 0 && N / kBN > cus && N / kBN >= 128;
}

// Workgroups per 16-column tile: a split of the reduction when the tiles
// alone leave most of the chip idle and there are enough rows to amortise
// the partial exchange (measured: the exchange costs more than it saves at
// one or two 16-row tiles).
int linear_splits(int M, int N, int K) {
  const int tiles = N / kBN;
  if (M < 32 || M > kMaxRows || tiles >= 128) return 1;
  int ks = 256 / tiles;
  ks = ks > kMaxSplits ? kMaxSplits : (ks < 1 ? 1 : ks);
  while (ks > 1 && K < ks * kLinWaves * 64) --ks;  // every worker keeps a chunk of the larger size
  return ks;
}

// The dispatch of one call: tile width first, then the split count, which
// only the 16-column tiles take (the 8- and 32-column kernels deal the
// reduction to one workgroup's 8 waves and never merge partials).
struct LinPlan {
  int cols;    // output columns per workgroup: 8, 16 or 32
  int ks;      // workgroups per 16-column tile (split reduction), 1 otherwise
  bool small;  // half chunks (and two workgroups per CU where registers allow)
};

LinPlan linear_plan(int M, int N, int K, bool norm, int epi, int cus) {
  const int gy = (M + kMaxRows - 1) / kMaxRows;
  if (linear_wide_tiles(N, epi, cus)) return {32, 1, M <= 32 && (int64_t)(N / 32) * gy > cus};
  if (linear_quarter_tiles(M, N, norm, epi, cus)) return {4, 1, false};
  if (linear_half_tiles(M, N, norm, epi)) return {8, 1, (int64_t)(N / 8) * gy > cus};
  const int ks = linear_splits(M, N, K);
  return {16, ks, (int64_t)(N / kBN) * gy * ks > cus};
}

size_t linear_counter_bytes() { return (size_t)kMaxCounterTiles * sizeof(unsigned); }

size_t linear_ws_bytes(int ks, int N) {
  if (ks <= 1) return 0;
  const size_t tiles = (size_t)(N / kBN);
  return linear_counter_bytes() + tiles * ks * kMaxRows * kBN * sizeof(float);
}

template <int MT, int BNV, bool SMALL>
int launch_linear_tiles(const LinearArgs& a, bool norm, int epi, dim3 grid, hipStream_t s) {
#define NSV_LIN(NORM, EPI) \
  hipLaunchKernelGGL((linear_kernel<MT, NORM, EPI, SMALL, BNV>), grid, dim3(kLinThreads), 0, s, a)
  if constexpr (BNV == 32) {  // SwiGLU only
    if (norm) NSV_LIN(true, 1);
    else NSV_LIN(false, 1);
  } else if constexpr (BNV <= 8) {  // plain or residual, no prologue
    if (epi == 0) NSV_LIN(false, 0);
    else NSV_LIN(false, 2);
  } else if (norm) {
    if (epi == 0) NSV_LIN(true, 0);
    else if (epi == 1) NSV_LIN(true, 1);
    else NSV_LIN(true, 2);
  } else {
    if (epi == 0) NSV_LIN(false, 0);
    else if (epi == 1) NSV_LIN(false, 1);
    else NSV_LIN(false, 2);
  }
#undef NSV_LIN
  return nsv_launch_status();
}

template <int MT>
int launch_linear(const LinearArgs& a, const LinPlan& p, bool norm, int epi, hipStream_t s) {
  const dim3 grid(a.N / p.cols, (a.M + kMaxRows - 1) / kMaxRows, p.ks);
  if (p.cols == 32) {
    return p.small ? launch_linear_tiles<MT, 32, true>(a, norm, epi, grid, s)
                   : launch_linear_tiles<MT, 32, false>(a, norm, epi, grid, s);
  }
  if constexpr (MT <= 2) {  // 4- and 8-column tiles take at most 31 rows
    if (p.cols == 4) return launch_linear_tiles<MT, 4, false>(a, norm, epi, grid, s);
    if (p.cols == 8) {
      return p.small ? launch_linear_tiles<MT, 8, true>(a, norm, epi, grid, s)
                     : launch_linear_tiles<MT, 8, false>(a, norm, epi, grid, s);
    }
  }
  if (p.cols != kBN) return NSV_ERR_UNSUPPORTED;
  return p.small ? launch_linear_tiles<MT, kBN, true>(a, norm, epi, grid, s)
                 : launch_linear_tiles<MT, kBN, false>(a, norm, epi, grid, s);
}


// ---------------------------------------------------------------------------
// Streaming projection for very wide outputs (the LM head: a vocabulary of
// 151,936 weight rows): y[M, N] = x[M, K] W[N, K]^T with the plain epilogue,
// for as many rows as the activations fit the LDS (M (K + 8) bf16).  One
// workgroup per CU, its activations staged in LDS once; each wave then
// streams whole 16-row weight tiles (tiles gw, gw + W, ... for global wave
// gw of W), every 256-element group of a tile's rows loaded straight into
// the MFMA A-operand layout (lane (g4, c): row c, 8 elements at 32 s + 8 g4)
// while the previous group is multiplied, so each wave keeps two groups (16
// KiB) in flight with no workgroup barrier after the staging and no
// cross-wave reduction: a wave owns a tile's whole reduction.
// ---------------------------------------------------------------------------
constexpr int kStreamWaves = 8;
constexpr int kStreamKG = 256;                 // reduction elements per load group: 8 MFMA k-steps
constexpr int kStreamLds = 160 * 1024;         // LDS bytes a workgroup may hold (gfx950)

struct StreamArgs {
  const uint16_t* x;  // [M, K]
  const uint16_t* w;  // [N, K]
  uint16_t* y;        // [M, N]
  int M, N, K;
  int tiles;          // N / 16
};

// PACKED: the weights in the layout nsv_lm_head_pack writes, where each
// load instruction of a wave reads 1 KiB in a row (below).
template <int MT, int NG, bool PACKED>  // NG = K / 256 load groups per tile
__global__ __launch_bounds__(kStreamWaves * 64, 1) void stream_linear_kernel(StreamArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char xs_raw[];  // [M][K + 8] bf16
  __asm__ volatile("" ::"s"(a.x), "s"(a.w), "s"(a.y), "s"(a.M), "s"(a.N), "s"(a.K), "s"(a.tiles));
  constexpr int K = NG * kStreamKG;
  constexpr int XSTR = K + 8;  // staged row stride (elements): the 16 rows of a B-operand read fall in distinct banks
  uint16_t* xs = reinterpret_cast<uint16_t*>(xs_raw);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, c = lane & 15;
  const int M = a.M;
  const int nwaves = gridDim.x * kStreamWaves;
  const int gw = blockIdx.x * kStreamWaves + w;
  const int my_tiles = gw < a.tiles ? (a.tiles - gw + nwaves - 1) / nwaves : 0;  // uniform

  // the activations, 16-byte chunks tid, tid + 512, ..., 8 loads per batch
  const int chunks = M * (K / 8);
  for (int i0 = 0; i0 < chunks; i0 += 8 * kStreamWaves * 64) {
    u32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = min(i0 + j * kStreamWaves * 64 + tid, chunks - 1);
      v[j] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)i * 8);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0 + j * kStreamWaves * 64 + tid;
      if (i < chunks) {
        const int m = i / (K / 8), k8 = i - m * (K / 8);
        *reinterpret_cast<u32x4*>(xs + m * XSTR + k8 * 8) = v[j];
      }
    }
  }
  __syncthreads();
  if (my_tiles == 0) return;

  // The weights through a buffer resource of exactly N x K elements (the
  // plan admits this kernel only a MiB below 2^31 bytes).  wrow(i): byte offset
  // of this lane's row of the wave's tile i; past its last tile the offset
  // lies at the resource's end, so the group the loop issues ahead after
  // the last tile returns zeros without a memory access (it used to re-read
  // the last tile, and the wave's end waited for those loads).
  const __amdgpu_buffer_rsrc_t wrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.w), (short)0, (int)((int64_t)a.N * K * 2), 0x00020000);
  const int w_end = (int)((int64_t)a.N * K * 2);
  // Row-major [N, K]: load s of a group gives each of the tile's 16 rows 64
  // bytes, half of a 128-byte line, and the next load the other half.
  // Packed: the tile's 16 rows stored in exactly this load order, so load s
  // is 1 KiB in a row (whole lines).  MI355X, graph-replayed, the 0.6B head
  // (311 MB): 58-60 -> 51 us at 9 rows, 77 -> 65 at 72; the 8B head: 232 ->
  // 194 us at 9 rows.
  constexpr int LSTEP = PACKED ? 1024 : 64;                     // bytes between a group's loads
  constexpr int GSTEP = PACKED ? 8 * 1024 : kStreamKG * 2;      // bytes between a tile's groups
  auto wrow = [&](int i) {
    if (i >= my_tiles) return w_end;
    const int t = gw + i * nwaves;
    return PACKED ? t * 16 * K * 2 + lane * 16 : (((t * 16 + c) * K) + 8 * g4) * 2;
  };
  auto issue = [&](u32x4 (&buf)[8], int off) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
      buf[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, off + LSTEP * s, 0, kCpolNt));
  };
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  int brow[MT];  // staged row of each m-tile's B operand (rows past M read row M - 1; never stored)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) brow[mt] = min(mt * 16 + c, M - 1) * XSTR + 8 * g4;
  auto compute = [&](const u32x4 (&buf)[8], int kg) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4 bv = *reinterpret_cast<const u32x4*>(xs + brow[mt] + kg * kStreamKG + 32 * s);
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(to_bf16x8(buf[s]), to_bf16x8(bv), acc[mt], 0, 0, 0);
      }
    }
  };
  // y through a buffer resource of exactly M rows: the stores of rows past M
  // fall outside it and are dropped, so every store is unconditional (a
  // store under a branch leaves the compiler's wait counts inexact)
  const __amdgpu_buffer_rsrc_t yr =
      __builtin_amdgcn_make_buffer_rsrc(a.y, (short)0, (int)((int64_t)M * a.N * 2), 0x00020000);
  u32x4 A[8], B[8];
  issue(A, wrow(0));
  for (int i = 0; i < my_tiles; ++i) {
    const int p = wrow(i);
    const int pn = wrow(i + 1);
    // (scheduling barriers keep each group's 8 loads together and after the
    // multiplies that free their registers: the compiler otherwise spreads
    // them between the multiplies, reusing registers of loads in flight)
#pragma unroll
    for (int kg = 0; kg < NG; kg += 2) {
      __builtin_amdgcn_sched_barrier(0);
      issue(B, p + (kg + 1) * GSTEP);
      __builtin_amdgcn_sched_barrier(0);
      compute(A, kg);
      __builtin_amdgcn_sched_barrier(0);
      issue(A, kg + 2 < NG ? p + (kg + 2) * GSTEP : pn);
      __builtin_amdgcn_sched_barrier(0);
      compute(B, kg + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    // lane (g4, c) holds y[16 mt + c][16 t + 4 g4 .. + 3]
    const int t = gw + i * nwaves;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + c;
      const uint32_t lo = pack_bf16x2(acc[mt][0], acc[mt][1]), hi = pack_bf16x2(acc[mt][2], acc[mt][3]);
      const unsigned off = (unsigned)(((int64_t)m * a.N + t * 16 + 4 * g4) * 2);
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2v, make_uint2(lo, hi)), yr, (int)off, 0, 0);
      acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last (unused, out-of-range) group's loads
}

// Streaming kernel for a wide plain projection: at least four 16-row weight
// tiles per wave (8 waves per CU), a reduction of 1024, 2048 or 4096
// elements, and activations that fit the LDS.
bool stream_wide(int M, int N, int K, bool norm, int epi, int cus) {
  return !norm && epi == 0 && M >= 1 && M <= kMaxRows && (K == 1024 || K == 2048 || K == 4096) &&
         (int64_t)(N / kBN) >= 32LL * cus && (int64_t)M * (K + 8) * 2 <= kStreamLds &&
         (int64_t)M * N * 2 < ((int64_t)1 << 31) &&
         (int64_t)N * K * 2 <= ((int64_t)1 << 31) - (1 << 20);  // weight byte offsets (and one group past the end) fit an int
}

template <int MT, int NG, bool PACKED>
int launch_stream(const StreamArgs& a, int cus, hipStream_t s) {
  static int attr[64] = {0};  // per device: the dynamic LDS limit raised once
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return NSV_ERR_UNSUPPORTED;
  if (!attr[dev]) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&stream_linear_kernel<MT, NG, PACKED>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kStreamLds) != hipSuccess)
      return nsv_launch_status();
    attr[dev] = 1;
  }
  const size_t lds = (size_t)a.M * (a.K + 8) * 2;
  hipLaunchKernelGGL((stream_linear_kernel<MT, NG, PACKED>), dim3(cus), dim3(kStreamWaves * 64), lds, s, a);
  return nsv_launch_status();
}

template <int MT, bool PACKED>
int launch_stream_k(const StreamArgs& a, int cus, hipStream_t s) {
  switch (a.K) {
    case 1024: return launch_stream<MT, 4, PACKED>(a, cus, s);
    case 2048: return launch_stream<MT, 8, PACKED>(a, cus, s);
    default: return launch_stream<MT, 16, PACKED>(a, cus, s);  // 4096 (stream_wide admits no other)
  }
}

template <bool PACKED>
int launch_stream_rows(const StreamArgs& sa, int cus, hipStream_t st) {
  switch ((sa.M + 15) / 16) {
    case 1: return launch_stream_k<1, PACKED>(sa, cus, st);
    case 2: return launch_stream_k<2, PACKED>(sa, cus, st);
    case 3: return launch_stream_k<3, PACKED>(sa, cus, st);
    case 4: return launch_stream_k<4, PACKED>(sa, cus, st);
    default: return launch_stream_k<5, PACKED>(sa, cus, st);
  }
}

// The packed LM-head layout: 16-byte chunk q = ((t NG + kg) 8 + s) 64 + l of
// the output holds W[16 t + (l & 15)][256 kg + 32 s + 8 (l >> 4) .. + 7]:
// tile t's 16 rows, load group kg, load s, lane l, in the streaming kernel's
// MFMA operand order.  One thread per chunk.
__global__ __launch_bounds__(256) void lm_head_pack_kernel(const u32x4* __restrict__ w, u32x4* __restrict__ out,
                                                           int64_t chunks, int K) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= chunks) return;
  const int l = (int)(q & 63), ld = (int)((q >> 6) & 7);
  const int64_t rest = q >> 9;
  const int ng = K / kStreamKG;
  const int64_t t = rest / ng;
  const int kg = (int)(rest - t * ng);
  const int64_t src = ((t * 16 + (l & 15)) * K + kg * kStreamKG + 32 * ld + 8 * (l >> 4)) / 8;
  out[q] = w[src];
}


// ---------------------------------------------------------------------------
// Decode-shaped projection (at most kDecodeRows rows, e.g. a drafter's one or
// two rows per sequence): one wave per output column (SwiGLU: per gate/up
// row pair), the whole reduction in that wave -- its weight row, the
// activation rows and (RMSNorm prologue) the norm weight and the producer's
// partial sums all loaded in one round trip, fp32 dot products on the VALU
// summed across the wave with DPP, and the epilogue in the same wave.  No
// LDS staging, no cross-wave reduction (except the residual epilogue's
// partial sums of squares, one per workgroup of 4 columns).  The operations
// per output are those of the tiled kernel (W' = bf16(W * norm_w), one bf16
// rounding of each product, the same epilogues); the reduction order is its
// own.
// ---------------------------------------------------------------------------
constexpr int kDecodeRows = 2;
constexpr int kDecodeWaves = 4;  // columns per workgroup (one partial-sum slot each with the residual epilogue)

template <int EPI, bool NORM, int KL, int MR>  // KL = K / 512 16-byte chunks per lane; MR rows (<= kDecodeRows)
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_linear_kernel(LinearArgs a) {
  __asm__ volatile("" ::"s"(a.x), "s"(a.norm_w), "s"(a.ss_in), "s"(a.nss_in), "s"(a.eps), "s"(a.w), "s"(a.y),
                   "s"(a.resid), "s"(a.ss_out), "s"(a.M), "s"(a.N), "s"(a.K));
  __shared__ float ssq[kDecodeWaves][MR];
  constexpr int K = KL * 512;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ncols = EPI == 1 ? a.N / 2 : a.N;
  const int col_raw = blockIdx.x * kDecodeWaves + w;
  const int col = min(col_raw, ncols - 1);  // (past the last column: read the last, store nothing)
  const int M = a.M;
  // ---- every load, one round trip (the residual elements first: nothing
  // before them is waited for)
  uint32_t rres[MR];
  if constexpr (EPI == 2) {
#pragma unroll
    for (int m = 0; m < MR; ++m) rres[m] = a.resid[(int64_t)min(m, M - 1) * a.N + col];
  }
  u32x4 wv[KL], uv[EPI == 1 ? KL : 1], xv[MR][KL], nv[NORM ? KL : 1];
  const uint16_t* wr = a.w + (int64_t)col * K + lane * 8;
#pragma unroll
  for (int i = 0; i < KL; ++i) wv[i] = load16_stream(wr + i * 512);
  if constexpr (EPI == 1) {
    const uint16_t* ur = a.w + (int64_t)(a.N / 2 + col) * K + lane * 8;
#pragma unroll
    for (int i = 0; i < KL; ++i) uv[i] = load16_stream(ur + i * 512);
  }
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int i = 0; i < KL; ++i)
      xv[m][i] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)min(m, M - 1) * K + i * 512 + lane * 8);
  float ssv[NORM ? MR : 1][4];
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < KL; ++i) nv[i] = *reinterpret_cast<const u32x4*>(a.norm_w + i * 512 + lane * 8);
    // slots lane, lane + 64, ... of each row (at most 256 slots: the host's bound)
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        ssv[m][u] = a.ss_in[(int64_t)min(lane + 64 * u, a.nss_in - 1) * a.M + min(m, M - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);  // (every load above is issued before any of them is used)
  // (used here, so that no load is moved under the selects and branches below)
  if constexpr (NORM) {
#pragma unroll
    for (int m = 0; m < MR; ++m) __asm__ volatile("" ::"v"(ssv[m][0]), "v"(ssv[m][1]), "v"(ssv[m][2]), "v"(ssv[m][3]));
  }
  if constexpr (EPI == 2) {
#pragma unroll
    for (int m = 0; m < MR; ++m) __asm__ volatile("" ::"v"(rres[m]));
  }
  // ---- dot products: lane holds elements 512 i + 8 lane .. + 7
  auto dot = [&](const u32x4 (&wrow)[KL], int m) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < KL; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float wf = bfv(wrow[i][q], h);
          if constexpr (NORM) wf = bf16_bits_to_f32(f32_to_bf16_bits(wf * bfv(nv[i][q], h)));
          acc = fmaf(bfv(xv[m][i][q], h), wf, acc);
        }
    return wave_sum(acc);
  };
  float inv[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    inv[m] = 1.f;
    if constexpr (NORM) {
      float t = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) t += lane + 64 * u < a.nss_in ? ssv[m][u] : 0.f;
      inv[m] = rsqrtf(wave_sum(t) / (float)K + a.eps);
    }
  }
  const bool live = col_raw < ncols;  // uniform
  if constexpr (EPI == 1) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float g = bf16_bits_to_f32(f32_to_bf16_bits(dot(wv, m) * inv[m]));
      const float u = bf16_bits_to_f32(f32_to_bf16_bits(dot(uv, m) * inv[m]));
      if (live && lane == 0 && m < M) a.y[(int64_t)m * ncols + col] = f32_to_bf16_bits(g / (1.f + __expf(-g)) * u);
    }
  } else {
    float ssm[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = bf16_bits_to_f32(f32_to_bf16_bits(dot(wv, m) * inv[m]));
      ssm[m] = 0.f;
      if constexpr (EPI == 2) {
        v = bf16_bits_to_f32(f32_to_bf16_bits(v + bf16_bits_to_f32(rres[m] & 0xffffu)));  // the residual stream is bf16
        ssm[m] = live ? v * v : 0.f;
        if (live && lane == 0 && m < M) a.resid[(int64_t)m * a.N + col] = f32_to_bf16_bits(v);
      } else {
        if (live && lane == 0 && m < M) a.y[(int64_t)m * a.N + col] = f32_to_bf16_bits(v);
      }
    }
    if constexpr (EPI == 2) {
      // the workgroup's 4 columns: one partial sum of squares per row, added in wave order
      if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) ssq[w][m] = ssm[m];
      }
      __syncthreads();
      if (threadIdx.x < MR && (int)threadIdx.x < M) {
        const int m = threadIdx.x;
        float t = 0.f;
#pragma unroll
        for (int ww = 0; ww < kDecodeWaves; ++ww) t += ssq[ww][m];
        a.ss_out[(int64_t)blockIdx.x * a.M + m] = t;
      }
    }
  }
}

template <int EPI, bool NORM, int KL>
int launch_decode_k(const LinearArgs& a, hipStream_t s) {
  const int ncols = EPI == 1 ? a.N / 2 : a.N;
  const dim3 grid((ncols + kDecodeWaves - 1) / kDecodeWaves);
  if (a.M <= 1) hipLaunchKernelGGL((decode_linear_kernel<EPI, NORM, KL, 1>), grid, dim3(kDecodeWaves * 64), 0, s, a);
  else hipLaunchKernelGGL((decode_linear_kernel<EPI, NORM, KL, 2>), grid, dim3(kDecodeWaves * 64), 0, s, a);
  return nsv_launch_status();
}

template <int EPI, bool NORM>
int launch_decode(const LinearArgs& a, hipStream_t s) {
  switch (a.K / 512) {
    case 2: return launch_decode_k<EPI, NORM, 2>(a, s);
    case 4: return launch_decode_k<EPI, NORM, 4>(a, s);
    case 6: return launch_decode_k<EPI, NORM, 6>(a, s);
    default: return launch_decode_k<EPI, NORM, 8>(a, s);
  }
}

}  // namespace

extern "C" {

int nsv_linear_ss_rows(int M, int N, int K, int has_norm) {
  if (M <= 0 || N <= 0 || K <= 0 || N % kBN) return 0;
  if (linear_quarter_tiles(M, N, has_norm != 0, 2, lin_device_cus())) return N / 4;
  return linear_half_tiles(M, N, has_norm != 0, 2) ? N / 8 : N / kBN;
}

size_t nsv_linear_workspace_size(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0 || N % kBN) return 0;
  return linear_ws_bytes(linear_splits(M, N, K), N);
}

int nsv_linear_plan(int M, int N, int K, int has_norm, int epilogue, int cus, int* tile_cols, int* splits,
                    int* half_chunks) {
  if (M <= 0 || N <= 0 || K <= 0 || epilogue < 0 || epilogue > 2 || N % kBN || K % 8) return NSV_ERR_ARG;
  const int c = cus > 0 ? cus : lin_device_cus();
  if (stream_wide(M, N, K, has_norm != 0, epilogue, c)) {  // whole 16-row weight tiles per wave
    if (tile_cols) *tile_cols = kBN;
    if (splits) *splits = 1;
    if (half_chunks) *half_chunks = 2;
    return NSV_OK;
  }
  const LinPlan p = linear_plan(M, N, K, has_norm != 0, epilogue, c);
  if (tile_cols) *tile_cols = p.cols;
  if (splits) *splits = p.ks;
  if (half_chunks) *half_chunks = p.small ? 1 : 0;
  return NSV_OK;
}

int nsv_linear_decode_ss_rows(int M, int N) {
  if (M <= 0 || M > kDecodeRows || N <= 0 || N % kBN) return 0;
  return (N + kDecodeWaves - 1) / kDecodeWaves;
}

int nsv_linear_decode(const void* x, const void* norm_w, const float* ss_in, int nss_in, float eps, const void* weight,
                      void* y, void* resid, float* ss_out, int M, int N, int K, int epilogue, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || epilogue < 0 || epilogue > 2) return NSV_ERR_ARG;
  if (M == 0) return NSV_OK;
  if (M > kDecodeRows || N % kBN || (K != 1024 && K != 2048 && K != 3072 && K != 4096)) return NSV_ERR_UNSUPPORTED;
  if (!x || !weight) return NSV_ERR_ARG;
  if (norm_w && (!ss_in || nss_in <= 0)) return NSV_ERR_ARG;
  if (norm_w && nss_in > 256) return NSV_ERR_UNSUPPORTED;
  if (epilogue == 2 ? (!resid || !ss_out) : !y) return NSV_ERR_ARG;
  LinearArgs a{};
  a.x = (const uint16_t*)x;
  a.norm_w = (const uint16_t*)norm_w;
  a.ss_in = ss_in;
  a.nss_in = nss_in;
  a.eps = eps;
  a.w = (const uint16_t*)weight;
  a.y = (uint16_t*)y;
  a.resid = (uint16_t*)resid;
  a.ss_out = ss_out;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ks = 1;
  hipStream_t s = (hipStream_t)stream;
  const bool norm = norm_w != nullptr;
  if (epilogue == 0) return norm ? launch_decode<0, true>(a, s) : launch_decode<0, false>(a, s);
  if (epilogue == 1) return norm ? launch_decode<1, true>(a, s) : launch_decode<1, false>(a, s);
  return norm ? launch_decode<2, true>(a, s) : launch_decode<2, false>(a, s);
}

int nsv_linear(const void* x, const void* norm_w, const float* ss_in, int nss_in, float eps, const void* weight,
               void* y, void* resid, float* ss_out, int M, int N, int K, int epilogue, void* workspace,
               size_t workspace_bytes, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || epilogue < 0 || epilogue > 2) return NSV_ERR_ARG;
  if (M == 0) return NSV_OK;
  if (N % kBN || K % 8 || M > 65535 * kMaxRows) return NSV_ERR_UNSUPPORTED;
  if (!x || !weight) return NSV_ERR_ARG;
  if (norm_w && (!ss_in || nss_in <= 0)) return NSV_ERR_ARG;
  if (epilogue == 2 ? (!resid || !ss_out) : !y) return NSV_ERR_ARG;
  const bool norm = norm_w != nullptr;
  if (stream_wide(M, N, K, norm, epilogue, lin_device_cus())) {
    const StreamArgs sa{(const uint16_t*)x, (const uint16_t*)weight, (uint16_t*)y, M, N, K, N / kBN};
    return launch_stream_rows<false>(sa, lin_device_cus(), (hipStream_t)stream);
  }
  const LinPlan p = linear_plan(M, N, K, norm, epilogue, lin_device_cus());
  const size_t need = linear_ws_bytes(p.ks, N);
  if (need && (!workspace || workspace_bytes < need)) return NSV_ERR_WORKSPACE;
  const size_t cnt = linear_counter_bytes();
  LinearArgs a{(const uint16_t*)x, (const uint16_t*)norm_w, ss_in, nss_in, eps, (const uint16_t*)weight,
               (uint16_t*)y, (uint16_t*)resid, ss_out, M, N, K, p.ks,
               need ? (float*)((char*)workspace + cnt) : nullptr, need ? (unsigned*)workspace : nullptr};
  hipStream_t s = (hipStream_t)stream;
  switch ((min(M, kMaxRows) + 15) / 16) {
    case 1: return launch_linear<1>(a, p, norm, epilogue, s);
    case 2: return launch_linear<2>(a, p, norm, epilogue, s);
    case 3: return launch_linear<3>(a, p, norm, epilogue, s);
    case 4: return launch_linear<4>(a, p, norm, epilogue, s);
    default: return launch_linear<5>(a, p, norm, epilogue, s);
  }
}

int nsv_lm_head_rows(int N, int K) {
  if (N <= 0 || N % kBN || (K != 1024 && K != 2048 && K != 4096)) return 0;
  const int rows = min(kMaxRows, kStreamLds / ((K + 8) * 2));
  if (!stream_wide(1, N, K, false, 0, lin_device_cus()) || (int64_t)rows * N * 2 >= ((int64_t)1 << 31)) return 0;
  return rows;
}

int nsv_lm_head_pack(const void* weight, void* packed, int N, int K, void* stream) {
  if (!weight || !packed || N <= 0 || K <= 0) return NSV_ERR_ARG;
  if (N % kBN || (K != 1024 && K != 2048 && K != 4096)) return NSV_ERR_UNSUPPORTED;
  if (weight == packed) return NSV_ERR_ARG;
  const int64_t chunks = (int64_t)N * K / 8;
  hipLaunchKernelGGL(lm_head_pack_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4*)weight, (u32x4*)packed, chunks, K);
  return nsv_launch_status();
}

int nsv_lm_head(const void* x, const void* packed, void* y, int M, int N, int K, void* stream) {
  if (M < 0 || N <= 0 || K <= 0) return NSV_ERR_ARG;
  if (M == 0) return NSV_OK;
  if (!x || !packed || !y) return NSV_ERR_ARG;
  if (M > nsv_lm_head_rows(N, K)) return NSV_ERR_UNSUPPORTED;
  const StreamArgs sa{(const uint16_t*)x, (const uint16_t*)packed, (uint16_t*)y, M, N, K, N / kBN};
  return launch_stream_rows<true>(sa, lin_device_cus(), (hipStream_t)stream);
}

}  // extern "C"
