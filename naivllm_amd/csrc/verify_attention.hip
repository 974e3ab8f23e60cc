// Paged multi-token verify attention and paged KV scatter for gfx950.
//
// Behaviour follows the reference's Triton path
// (src/myvllm/layers/attention.py:522-668 verify, :9-112 KV store); the
// decomposition is this library's own.  Common to the bf16 kernels:
//
//   * a workgroup serves one (sequence, kv-head) pair -- every query row of
//     its GQA group -- from one read of the pair's K/V (the reference
//     re-reads K/V once per query head);
//   * the group's query rows are packed into 16-row MFMA tiles: rows
//     m = g * QL + t for group member g and verify row t;
//   * S^T = K Q^T is computed so that the MFMA result layout is directly the
//     B operand of O^T = V^T P^T (no register shuffles between the two
//     products); V is staged through LDS and read back with gfx950's
//     transposing LDS read;
//   * every K/V load of a tile is unconditional (missing keys read a mapped
//     row), so the compiler's wait counts stay exact across the pipeline; a
//     tile with no key at all issues no load (in the key-split kernel from a
//     wave's second tile on), so no dummy loads queue beside real ones.
//
// Two bf16 decompositions, chosen by make_plan:
//   * key-split (verify_attn_ks_kernel): workgroup = (pair, key split), full
//     head dim; splits of a pair merge in-kernel (the last split to finish
//     combines the partials, exchanged with agent-scope loads and stores);
//   * d-sliced (verify_attn_bf16_kernel): workgroup = (pair, head-dim slice,
//     key split); every slice recomputes the scores and reads the pair's K
//     through its own L1 (shared in L2); the key splits of a slice, when
//     used, merge in-kernel like the key-split kernel's (the last of them to
//     finish), or in a second kernel past the arrival counters' capacity.
// The fp32 kernel (the 1e-5 contract) uses VALU dot products.

#include "common.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace {

constexpr int kTile = 32;   // keys per wave iteration
constexpr int kBf16Waves = 8;  // waves per workgroup (d-sliced bf16 kernel)
#ifndef NSV_KS_WAVES
#define NSV_KS_WAVES 8
#endif
constexpr int kKsWaves = NSV_KS_WAVES;  // waves per workgroup of the key-split kernel (two workgroups per CU)
constexpr int kMaxSplitPages = 1024;  // block-table entries of one split staged in LDS
// Pairs of the key-split kernel's arrival-counter area at the front of the
// workspace.  The area has one fixed size, so every call finds its counters
// at the same place, zero, whatever the previous call's shape was.
constexpr int kMaxCounterPairs = 16384;
// Counter slot of a pair: pairs 0..255 each get their own 256-byte line
// (device-scope atomics on one line serialise, ~20 ns apiece), and pair
// p + 256 k shares p's line.
__device__ __forceinline__ int counter_slot(int pair) { return ((pair & 255) << 6) | (pair >> 8); }


// Pipeline depth of the d-sliced bf16 kernel.  Its slices re-read the pair's
// K through L1, whose fill rate bounds it, and deeper pipelines only add
// pressure there: on MI355X at config 2, 2 stages take 20.6 us, 3 21.3 us,
// 4 23.2 us.  So 2, the floor of the register estimate used for the
// key-split kernel below.
#ifndef NSV_DSLICE_STAGES
#define NSV_DSLICE_STAGES 2
#endif
constexpr int bf16_stages(int MT, int DH, int DC, bool UPAGE) {
  // register estimate of a deeper pipeline (tiles of 40 VGPRs beyond a fixed part), floored at 2
  const int KS = DH / 32, DT = DC / 16, VL = 32 * (DC / 8) / 64;
  const int fixed = 20 + MT * (KS * 4 + DT * 4 + 12) + (UPAGE ? 32 : 64);
  const int fit = (256 - fixed) / (8 * KS + 4 * VL);
  const int want = NSV_DSLICE_STAGES;
  return want < 2 ? 2 : (want > fit ? (fit < 2 ? 2 : fit) : want);
}
constexpr float kNegInf = -__builtin_inff();
// how far (log2 domain) a row's running maximum may pass its exponent reference
// before the key-split kernel moves the reference (weights stay <= 2^8)
constexpr float kRefSlack = 8.f;

// Timeline stamps (a build knob: libnaivspec_stamp.so is built with
// NSV_STAMP=1; the default library has no stamp code).  Thread 0 of every
// workgroup of a stamped launch writes the 100 MHz constant clock
// (s_memrealtime, 10 ns ticks, one clock for the whole chip) at numbered
// points of the kernel into its row of kStampSlots words, and its XCD id
// into the last word.
#ifndef NSV_STAMP
#define NSV_STAMP 0
#endif
constexpr int kStampSlots = 16;
constexpr int kStampMaxWgs = 4096;  // workgroups a stamped launch records

struct VerifyArgs {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_tables;
  const int64_t* context_lens;
  const int32_t* cu_seqlens_q;
  const int64_t* positions;
  void* out;
  float* part_ml;    // [B, Hkv, S, Mv, 2]  (running max, running sum), log2 domain
  float* part_o;     // [B, Hkv, S, Mv, D]  unnormalised split outputs
  unsigned* counters;  // [B, Hkv] splits of the pair done so far (key-split kernel; 0 between calls)
  float scale_log2;  // softmax scale * log2(e)
  int H, Hkv, G, bs_log2, max_blocks, QL, Mv, S, split_tokens, P8, npairs;
  int Gs, g0;        // query heads per kv head, and the first of the G this launch serves
  int dqc;           // head-dim slices per pair (d-sliced bf16 kernel)
  int ks_splits;     // key-split kernel: splits per sequence when split_tokens == 0
  int m_base;        // fp32 kernel: first query row (of the Mv) this launch serves
  int dmerge;        // d-sliced kernel: the pair's last workgroup merges its splits in-kernel (else a merge launch)
#if NSV_STAMP
  unsigned long long* stamps;  // [grid][kStampSlots] of this launch, or null
#endif
};

#if NSV_STAMP
#define NSV_STAMP_AT(a, slot)                                                                      \
  do {                                                                                             \
    if ((a).stamps && threadIdx.x == 0)                                                            \
      (a).stamps[((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * kStampSlots + (slot)] = __builtin_amdgcn_s_memrealtime();            \
  } while (0)
// hwreg(HW_REG_XCC_ID = 20, offset 0, 4 bits): the XCD the workgroup runs on
#define NSV_STAMP_XCC(a)                                                                           \
  do {                                                                                             \
    if ((a).stamps && threadIdx.x == 0)                                                            \
      (a).stamps[((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * kStampSlots + kStampSlots - 1] =                                     \
          (unsigned long long)(__builtin_amdgcn_s_getreg(20 | (3 << 11)) & 15);                    \
  } while (0)
#else
#define NSV_STAMP_AT(a, slot) \
  do {                        \
  } while (0)
#define NSV_STAMP_XCC(a) \
  do {                   \
  } while (0)
#endif

__device__ __forceinline__ u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }


// A float pair as one 64-bit agent-scope (device-coherent) relaxed atomic
// store: coherent across XCDs without cache maintenance instructions.
__device__ __forceinline__ void store_agent(uint64_t* p, float x, float y) {
  const uint64_t v = (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32);
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// A row's position (int64; every position a plan accepts, -1 included, fits
// 32 bits) read as the low word of the little-endian value.  A 64-bit load
// whose upper half is dead lets the compiler reuse that register while the
// load is in flight, and the reuse then waits for the load: a whole memory
// round trip before the first K/V load is issued.
__device__ __forceinline__ int load_pos(const int64_t* positions, int64_t row) {
  return reinterpret_cast<const int32_t*>(positions)[2 * row];
}

// Keys of sequence b the kernels visit: never past the block table's width,
// the bound the reference's chunk loop has (layers/attention.py:572).
// (A workgroup's per-sequence values are read by every lane and made
// wave-uniform: the compiler cannot prove on its own that memory the kernel
// also writes holds the same value for every lane, and would keep them per
// lane, each use as a scalar operand then a loop over the lanes' values.)
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
// The kernel arguments a kernel's first round trip needs, fetched in one
// batch at its start: the empty statements use them, so the compiler cannot
// defer one of their loads past the first use of another (each deferred load
// is a dependent round trip of its own before the first K/V load).
__device__ __forceinline__ void fetch_args(const VerifyArgs& a) {
  __asm__ volatile("" ::"s"(a.block_tables), "s"(a.context_lens), "s"(a.cu_seqlens_q), "s"(a.P8), "s"(a.npairs),
                   "s"(a.Hkv), "s"(a.max_blocks), "s"(a.bs_log2), "s"(a.split_tokens), "s"(a.dqc), "s"(a.ks_splits),
                   "s"(a.S), "s"(a.Mv), "s"(a.QL));
}
// The sequence's context length and query range, used here so that their
// loads stay ahead of every exit (a load whose value only a later block uses
// is otherwise moved into that block, behind the exit's branch).
__device__ __forceinline__ void pin_metadata(int64_t ctx, int q0, int q1) {
  __asm__ volatile("" ::"s"(ctx), "s"(q0), "s"(q1));
}

__device__ __forceinline__ int clamp_context(const VerifyArgs& a, int64_t ctx) {
  const int64_t cap = (int64_t)a.max_blocks << a.bs_log2;
  return uniform((int)(ctx < 0 ? 0 : (ctx < cap ? ctx : cap)));
}
__device__ __forceinline__ int context_len(const VerifyArgs& a, int b) { return clamp_context(a, a.context_lens[b]); }

// Keys per split of a sequence with ctx keys: the caller's fixed split, or
// (key-split kernel, automatic) ctx spread evenly over ks_splits splits in
// whole 16-key tiles.
__device__ __forceinline__ int split_len(const VerifyArgs& a, int ctx) {
  if (a.split_tokens > 0) return a.split_tokens;
  const int per = (ctx + a.ks_splits - 1) / a.ks_splits;
  return per <= 16 ? 16 : (per + 15) & ~15;
}

// Number of key splits sequence b actually uses (>= 1 so that an empty
// sequence still gets its rows written).
__device__ __forceinline__ int num_splits(const VerifyArgs& a, int ctx) {
  const int len = split_len(a, ctx);
  return ctx <= len ? 1 : (ctx + len - 1) / len;
}

__device__ __forceinline__ int split_len_ks(const VerifyArgs& a, int ctx) {
  if (a.split_tokens > 0) return a.split_tokens;
  const int per = div_small(ctx + a.ks_splits - 1, a.ks_splits);
  return per <= 16 ? 16 : (per + 15) & ~15;
}
__device__ __forceinline__ int num_splits_ks(int ctx, int len) { return ctx <= len ? 1 : div_small(ctx + len - 1, len); }

// Workgroup -> (split, pair) with every split of a (sequence, kv-head) pair
// on the same XCD (workgroups are dealt to the 8 XCDs round-robin), so the
// pair's shared query rows and partials stay in one L2.
__device__ __forceinline__ void decode_block(const VerifyArgs& a, int& split, int& pair) {
  const int i = blockIdx.x;
  const int y = i >> 3;
  split = y / a.P8;
  pair = (y - split * a.P8) * 8 + (i & 7);
}

// ---------------------------------------------------------------------------
// bf16 d-sliced kernel: 8 waves, MFMA 16x16x32.
// ---------------------------------------------------------------------------
// Cross-lane reductions over the four lanes c, c+16, c+32, c+48 that hold one
// query row's statistics, with gfx950's permlane swaps (VALU, no LDS round
// trip): permlane{16,32}_swap(x, x) returns {x[l], x[l ^ 16 or 32]}.
__device__ __forceinline__ float row_max4(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float row_sum4(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// gfx950 transposing LDS read: within each 16-lane group, lane i receives
// element (i % 4) of the 4-element rows addressed by lanes 4j + i/4, j = 0..3.
__device__ __forceinline__ uint2 lds_read_tr(const uint16_t* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

// Workgroup = (pair, slice dq of DC head dims, key split); its kBf16Waves
// waves take interleaved 32-key tiles of the split.  Every slice recomputes
// the scores (cheap: the kernel is HBM bound) and reads the pair's K from
// the L2 its sibling slices share (all workgroups of a pair sit on one XCD),
// so HBM sees each K/V byte about once while the grid has 128/DC times more
// workgroups than pairs — enough to cover the chip without key splits in
// the common case, which keeps the operator a single kernel.
//
// Each wave runs an NS-stage register pipeline: the loads of its next NS
// tiles are in flight while a tile computes (a short context's whole key
// range is in flight at once); two waves share each SIMD.  Block-
// table entries of the split are staged in LDS once.  UPAGE (block_size
// >= 32): a tile lies in one page, whose id is wave-uniform (scalar base
// address, 32-bit offsets).
//
// Softmax runs on raw scores: the running max m is taken over q.k, and
// p = 2^(q.k * scale*log2e - m * scale*log2e) is one FMA plus the hardware
// exp2 (results below 2^-126 flush to zero; their weight is negligible, as
// with the flush-to-zero exp of the reference's Triton kernel).  Tiles with
// every key present and below every real query row's position skip masking.
template <int MT, int DH, int DC, bool UPAGE, int NS>
__global__ __launch_bounds__(kBf16Waves * 64, 1) void verify_attn_bf16_kernel(VerifyArgs a) {
  constexpr int NW = kBf16Waves;
  constexpr int NT = NW * 64;
  constexpr int KS = DH / 32;    // k-steps of S^T = K Q^T
  constexpr int DT = DC / 16;    // 16-wide d tiles of this slice
  constexpr int MP = MT * 16;    // padded query rows
  constexpr int VCH = DC / 8;    // 16-byte chunks per key in the slice
  constexpr int VL = kTile * VCH / NSV_WAVE;  // 16-byte V loads per lane per tile
  constexpr int VSTR = DC + 16;  // staged V row stride (bf16): an odd multiple of 32 bytes,
                                 // so the transposing reads of 8 rows hit distinct banks
  constexpr int RSTR = DC + 4;   // merge-region row stride (floats)
  // UPAGE: K tiles are loaded as whole 2*DH-byte rows (CPR 16-byte chunks
  // per key, KPI keys per load) and reshaped through a per-wave LDS tile
  // into the MFMA operand layout, with chunk X of key r stored at slot
  // X ^ (r % CPR): the row-order writes and the operand-order reads then hit
  // distinct LDS banks.  (A CU ingests whole-row loads several times faster
  // than the operand order's 64 bytes from each of 16 keys 2 KB apart.)
  constexpr int CPR = DH / 8;
  constexpr int KPI = NSV_WAVE / CPR;
  constexpr int KROW = DH * 2;
  constexpr int KSTAGE = UPAGE ? NW * kTile * KROW : 0;
  constexpr int STAGE = NW * kTile * VSTR * 2 + KSTAGE;
  constexpr int MTILE_BYTES = NW * 16 * RSTR * 4;  // one m-tile of every wave's O
  constexpr int MTP0 = (72 * 1024) / MTILE_BYTES;
  constexpr int MTP = MTP0 < 1 ? 1 : (MTP0 > MT ? MT : MTP0);  // m-tiles merged per pass
  constexpr int MERGE = MTP * MTILE_BYTES;
  constexpr int SMEM = STAGE > MERGE ? STAGE : MERGE;

  // PARK: each wave parks its unscaled O slice and (max, sum) in LDS of its
  // own as soon as its tiles are done, while slower waves still stream; one
  // barrier later every output is the factor-weighted sum of the parked
  // slices.  Taken when the parking area fits beside the staging area.
  constexpr int PARK_FLOATS = NW * MP * RSTR;
  constexpr int QBYTES = MP * DH * 2;  // the query rows, staged once for the 8 waves
  constexpr bool PARK =
      SMEM + QBYTES + PARK_FLOATS * 4 + kMaxSplitPages * 4 + 2 * NW * MP * 4 + 3 * MP * 4 <= 159 * 1024;
  // One LDS block, the small arrays first: their addresses then fit the
  // 16-bit offset field of the LDS instructions.
  struct __attribute__((aligned(16))) Lds {
    float red_m[NW][MP];
    float red_l[NW][MP];
    float row_l[MP];
    float row_ms[MP];
    int row_pos[MP];
    int ds_last;
    int pages[kMaxSplitPages];
    // chunk X of query row m at slot X ^ (m % CPR): the 16 rows an operand
    // read touches fall in distinct banks
    __attribute__((aligned(16))) unsigned char q_lds[QBYTES];
    __attribute__((aligned(16))) unsigned char smem[SMEM];
    __attribute__((aligned(16))) float park[PARK ? PARK_FLOATS : 4];
  };
  __shared__ Lds lds;
  auto& red_m = lds.red_m;
  auto& red_l = lds.red_l;
  auto& row_l = lds.row_l;
  auto& row_ms = lds.row_ms;
  auto& row_pos = lds.row_pos;
  auto& ds_last = lds.ds_last;
  auto& pages = lds.pages;
  unsigned char* const smem = lds.smem;
  float* const park = lds.park;
  unsigned char* const q_lds = lds.q_lds;

  // ---- workgroup -> (pair, dq, split): grid (8 P8, dqc, splits), so
  // workgroup (z dqc + y) 8 P8 + x runs on XCD x % 8 -- every workgroup of a
  // pair on one XCD
  fetch_args(a);
  NSV_STAMP_AT(a, 0);  // entry
  NSV_STAMP_XCC(a);
  const int pair_raw = blockIdx.x;
  const int dq = blockIdx.y, split = blockIdx.z;
  // (the grid rounds the pair count up to a multiple of 8: workgroups past
  // the last pair, or past the table's keys, read clamped metadata and leave
  // once it is back -- an exit before those loads would put the kernel
  // arguments the loads need into a second, dependent round trip)
  const int pair = min(pair_raw, a.npairs - 1);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, c = lane & 15;
  const int b = div_small(pair, a.Hkv), hk = pair - b * a.Hkv;
  const int max_ctx = a.max_blocks << a.bs_log2;
  const int tok_begin = split * a.split_tokens;
  const int range_end = min(max_ctx, tok_begin + a.split_tokens);

  // ---- first round trip: the split's block-table slice, context length and
  // query-row range, all independent and issued before any is used
  // (entries past the slice read the row's last one and are not stored)
  const int pg0 = tok_begin >> a.bs_log2;
  const int npg = ((range_end - 1) >> a.bs_log2) - pg0 + 1;
  const int32_t* btrow = a.block_tables + (int64_t)b * a.max_blocks;
  constexpr int PPT = (kMaxSplitPages + NT - 1) / NT;
  int pv[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) pv[i] = btrow[min(pg0 + tid + i * NT, a.max_blocks - 1)];
  const int64_t ctx_raw = a.context_lens[b];
  const int q0 = uniform(a.cu_seqlens_q[b]);
  const int q1 = uniform(a.cu_seqlens_q[b + 1]);
  pin_metadata(ctx_raw, q0, q1);
  if (pair_raw >= a.npairs || tok_begin >= max_ctx) return;
  const int ctx = clamp_context(a, ctx_raw);
  const int qlen = q1 - q0;
  const int nsplit = num_splits(a, ctx);
  if (split >= nsplit || qlen < 0) return;  // uniform per workgroup
  NSV_STAMP_AT(a, 1);  // metadata back
  const int tok_end = min(ctx, range_end);
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int j = tid + i * NT;
    if (j < npg) pages[j] = pv[i];
  }

  // The query rows are loaded once per workgroup (16-byte chunks spread over
  // the threads), staged in LDS and read back by every wave as the B operand
  // of S^T: each wave loading them all put 8x the bytes through the CU's
  // intake ahead of the first tiles (b1 9.27 -> 8.89 us, 3k-key contexts
  // 10.39 -> 9.74).
  constexpr int QPASS = (MP * CPR + NT - 1) / NT;  // 16-byte query chunks per thread
  bf16x8 qB[MT][KS];
  u32x4 qt[QPASS];
  int qpos[MT];
  int qmin = 0x7fffffff;
  auto load_q = [&]() {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + c;
      const int g = div_small(m, a.QL), t = m - g * a.QL;
      const bool ok = (m < a.Mv) && (t < qlen);
      qpos[mt] = load_pos(a.positions, ok ? q0 + t : 0);
    }
#pragma unroll
    for (int i = 0; i < QPASS; ++i) {
      const int idx = tid + i * NT;
      const int m = idx / CPR, ch = idx % CPR;
      const int g = div_small(m, a.QL), t = m - g * a.QL;
      const bool ok = (idx < MP * CPR) && (m < a.Mv) && (t < qlen);
      const int row = ok ? q0 + t : 0;
      const int gg = ok ? g : 0;
      qt[i] = load16((const bf16_t*)a.q + ((int64_t)row * a.H + hk * a.Gs + a.g0 + gg) * DH + ch * 8);
    }
  };
  auto store_q = [&]() {
#pragma unroll
    for (int i = 0; i < QPASS; ++i) {
      const int idx = tid + i * NT;
      const int m = idx / CPR, ch = idx % CPR;
      if (idx < MP * CPR) *reinterpret_cast<u32x4*>(q_lds + m * (DH * 2) + ((ch ^ (m % CPR)) << 4)) = qt[i];
    }
  };
  auto read_q = [&]() {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + c;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qB[mt][ks] = as_bf16x8(*reinterpret_cast<const u32x4*>(q_lds + m * (DH * 2) + (((ks * 4 + g4) ^ (m % CPR)) << 4)));
    }
  };
  auto finish_positions = [&]() {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + c;
      const int g = div_small(m, a.QL), t = m - g * a.QL;
      const bool ok = (m < a.Mv) && (t < qlen);
      qpos[mt] = ok ? qpos[mt] : -1;
      if (qpos[mt] >= 0) qmin = min(qmin, qpos[mt]);
      if (w == 0 && g4 == 0) row_pos[m] = qpos[mt];
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) qmin = min(qmin, __shfl_xor(qmin, o, NSV_WAVE));
    qmin = __builtin_amdgcn_readfirstlane(qmin);
  };

  float m_run[MT], l_run[MT];  // running max of raw scores, running sum
  f32x4 acc[DT][MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    m_run[mt] = kNegInf;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const float sc = a.scale_log2;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const int tok_stride = a.Hkv * DH;  // elements between consecutive keys of a page
  const int64_t page_elems = (int64_t)tok_stride << a.bs_log2;
  const bf16_t* kbase = (const bf16_t*)a.k_cache + hk * DH;
  const bf16_t* vbase = (const bf16_t*)a.v_cache + hk * DH + dq * DC;
  uint16_t* vl = reinterpret_cast<uint16_t*>(smem) + w * kTile * VSTR;
  unsigned char* kl = smem + NW * kTile * VSTR * 2 + (UPAGE ? w * kTile * KROW : 0);
  __syncthreads();  // block-table slice visible

  const int ntiles = (tok_end - tok_begin + kTile - 1) / kTile;
  const int niter = (ntiles + NW - 1) / NW;  // same trip count in every wave

  struct Tile {
    u32x4 k[2][KS];  // UPAGE: whole rows, load j = t*KS + ks, lane -> (key KPI*j + lane/CPR, chunk lane%CPR);
                     // else the A operand: lane (g4, c) holds key 16*t + c, dims 32*ks + 8*g4 .. +7
    u32x4 v[VL];     // V slice rows, coalesced: chunk j*64 + lane = (key, 16-byte chunk)
    uint64_t kmask;  // keys of the tile that exist (inside the split, page mapped)
    int n0;
    int nvalid;      // UPAGE: the existing keys are exactly the first nvalid of the tile
  };

  // Issue every load of wave-tile `it`.  Masked keys read the row of a key
  // that exists (finite data, zero weight).  The first tile is always
  // issued (past the split's end it reads the pool's first row), so the
  // compiler's waits up to the query-staging barrier stay exact and the
  // barrier leaves it in flight; a later tile without any key (past the
  // split's end, or on an unmapped page) issues no load: such dummy loads,
  // a few per wave at these short splits, queued behind the real tiles in
  // the CU's address unit (b1: ~1.5 us before the waves merged).  (Loads at
  // an offset outside an empty buffer resource, which return zeros without
  // a memory access, still took that address-unit time: 9.2 -> 10.4 us.)
  auto issue = [&](Tile& T, int it, auto skip_empty) {
    T.n0 = tok_begin + (it * NW + w) * kTile;
    if constexpr (UPAGE) {
      int nvalid = min(max(tok_end - T.n0, 0), kTile);
      int pg = nvalid > 0 ? pages[(T.n0 >> a.bs_log2) - pg0] : -1;
      pg = __builtin_amdgcn_readfirstlane(pg);
      if (pg < 0) nvalid = 0;
      T.nvalid = nvalid;
      T.kmask = nvalid >= kTile ? 0xffffffffull : ((1ull << nvalid) - 1);
      if constexpr (decltype(skip_empty)::value) {
        if (nvalid == 0) return;  // uniform
      }
      // byte addressing: scalar page base + 32-bit lane offsets
      const size_t page_off = (size_t)(pg < 0 ? 0 : pg) * (size_t)page_elems * 2;
      const char* kp = (const char*)kbase + page_off;
      const char* vp = (const char*)vbase + page_off;
      const unsigned base_key = (unsigned)(T.n0 & bs_mask);
      const unsigned row_bytes = (unsigned)tok_stride * 2;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int r = KPI * (t * KS + ks) + lane / CPR;
          const unsigned off = (base_key + (r < nvalid ? r : 0)) * row_bytes + (lane % CPR) * 16;
          T.k[t][ks] = load16(kp + off);
        }
#pragma unroll
      for (int j = 0; j < VL; ++j) {
        const int id = j * NSV_WAVE + lane;
        const int r = id / VCH, ch = id - r * VCH;
        const unsigned off = (base_key + (r < nvalid ? r : 0)) * row_bytes + ch * 16;
        T.v[j] = load16_stream(vp + off);  // (K stays cached: the pair's other slices read it)
      }
    } else {
      const int n = T.n0 + lane;
      const int pg = (lane < kTile && n < tok_end) ? pages[(n >> a.bs_log2) - pg0] : -1;
      T.kmask = __ballot(pg >= 0);
      T.nvalid = 0;
      if constexpr (decltype(skip_empty)::value) {
        if (T.kmask == 0) return;  // uniform
      }
      const int first = T.kmask ? __builtin_ctzll(T.kmask) : 0;
      const int pg_first = __shfl(pg, first, NSV_WAVE);
      const int64_t dflt = T.kmask ? (int64_t)pg_first * page_elems + (int64_t)((T.n0 + first) & bs_mask) * tok_stride
                                   : 0;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = t * 16 + c;
        const int pk = __shfl(pg, r, NSV_WAVE);
        const int64_t row = ((T.kmask >> r) & 1) ? (int64_t)pk * page_elems + (int64_t)((T.n0 + r) & bs_mask) * tok_stride
                                                 : dflt;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) T.k[t][ks] = load16(kbase + row + g4 * 8 + ks * 32);
      }
#pragma unroll
      for (int j = 0; j < VL; ++j) {
        const int id = j * NSV_WAVE + lane;
        const int r = id / VCH, ch = id - r * VCH;
        const int pv = __shfl(pg, r, NSV_WAVE);
        const int64_t row = ((T.kmask >> r) & 1) ? (int64_t)pv * page_elems + (int64_t)((T.n0 + r) & bs_mask) * tok_stride
                                                 : dflt;
        T.v[j] = load16_stream(vbase + row + ch * 8);
      }
    }
  };

  auto compute = [&](const Tile& T) {
    if (T.kmask == 0) return;  // uniform: nothing of this tile exists
    // K operands: UPAGE reshapes the row-order tile through LDS (this wave's
    // rows; a wave's LDS ops complete in order)
    u32x4 kA[2][KS];
    if constexpr (UPAGE) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int r = KPI * (t * KS + ks) + lane / CPR;
          *reinterpret_cast<u32x4*>(kl + r * KROW + (((lane % CPR) ^ (r % CPR)) << 4)) = T.k[t][ks];
        }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int r = t * 16 + c;
          kA[t][ks] = *reinterpret_cast<const u32x4*>(kl + r * KROW + (((ks * 4 + g4) ^ (r % CPR)) << 4));
        }
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kA[t][ks] = T.k[t][ks];
    }
    // S^T tile: lane (g4, c), element i -> key 16*t + 4*g4 + i, query row 16*mt + c.
    f32x4 sacc[2][MT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kA[t][ks]), qB[mt][ks], sv, 0, 0, 0);
        sacc[t][mt] = sv;
      }
    // Stage the V slice (this wave's private LDS rows; LDS ops of one wave
    // complete in order).
#pragma unroll
    for (int j = 0; j < VL; ++j) {
      const int id = j * NSV_WAVE + lane;
      const int r = id / VCH, ch = id - r * VCH;
      *reinterpret_cast<u32x4*>(vl + r * VSTR + ch * 8) = T.v[j];
    }
    // Masked keys get -inf before any arithmetic (exact 0 weight).  Only the
    // tiles at a split's end or across a query row's position need it.
    const bool full = (T.kmask == 0xffffffffull) && (T.n0 + kTile - 1 <= qmin);
    if (!full) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = t * 16 + g4 * 4 + i;
          const bool exists = UPAGE ? (r < T.nvalid) : (bool)((T.kmask >> r) & 1);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            sacc[t][mt][i] = (exists && T.n0 + r <= qpos[mt]) ? sacc[t][mt][i] : kNegInf;
        }
    }
    bf16x8 pB[MT];
    float alpha[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float mx = __builtin_fmaxf(__builtin_fmaxf(sacc[0][mt][0], sacc[0][mt][1]), sacc[0][mt][2]);
      mx = __builtin_fmaxf(__builtin_fmaxf(mx, sacc[0][mt][3]), sacc[1][mt][0]);
      mx = __builtin_fmaxf(__builtin_fmaxf(mx, sacc[1][mt][1]), sacc[1][mt][2]);
      mx = __builtin_fmaxf(mx, sacc[1][mt][3]);
      mx = row_max4(mx);
      const float m_new = fmaxf(m_run[mt], mx);
      const float nb = (m_new == kNegInf) ? 0.f : -m_new * sc;  // exp2 bias
      alpha[mt] = __builtin_amdgcn_exp2f(fmaf(m_run[mt], sc, nb));
      float p[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[t][i] = __builtin_amdgcn_exp2f(fmaf(sacc[t][mt][i], sc, nb));
      const float sum = ((p[0][0] + p[0][1]) + (p[0][2] + p[0][3])) + ((p[1][0] + p[1][1]) + (p[1][2] + p[1][3]));
      l_run[mt] = fmaf(l_run[mt], alpha[mt], row_sum4(sum));
      m_run[mt] = m_new;
      // P^T as the B operand of O^T = V^T P^T, rounded to bf16 like the
      // reference's `p.to(v.dtype)`.  Element j covers key kmap(g4, j) =
      // 4*g4 + j (j < 4), 16 + 4*g4 + (j - 4) (j >= 4): the keys this lane's
      // S^T elements hold, so P needs no data movement.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pB[mt][i] = (bf16_t)p[0][i];
        pB[mt][4 + i] = (bf16_t)p[1][i];
      }
    }
    // rescale the accumulators only when some row's running max moved
    bool moved = false;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) moved |= alpha[mt] != 1.f;
    if (__ballot(moved)) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt][mt] *= alpha[mt];
    }
    __builtin_amdgcn_wave_barrier();
    // O^T += V^T P^T.  V^T operand of lane (g4, c): V[kmap(g4, j)][16*dt + c];
    // two transposing reads, each over rows kmap(g4, 4h .. 4h+3) with lane
    // k = c supplying row 4*g4 (+16 h) + k/4, columns 16*dt + 4*(k%4) .. +3.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint16_t* src = vl + (g4 * 4 + (c >> 2)) * VSTR + dt * 16 + (c & 3) * 4;
      const uint2 lo = lds_read_tr(src);
      const uint2 hi = lds_read_tr(src + 16 * VSTR);
      const bf16x8 vA = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[dt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vA, pB[mt], acc[dt][mt], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- NS-stage pipeline over this wave's tiles
  Tile T[NS];
  load_q();
  __builtin_amdgcn_sched_barrier(0);
  issue(T[0], 0, std::false_type{});
  __builtin_amdgcn_sched_barrier(0);
  finish_positions();
  store_q();
  lds_barrier();  // query rows visible; the first tile stays in flight
  read_q();
  __builtin_amdgcn_sched_barrier(0);
  // the later stages after the staging (an issue that may be skipped
  // before it would leave its waits inexact)
#pragma unroll
  for (int s = 1; s < NS; ++s) issue(T[s], s, std::true_type{});
  __builtin_amdgcn_sched_barrier(0);
  for (int it = 0; it < niter; it += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      compute(T[s]);
      if (it == 0 && s == 0) NSV_STAMP_AT(a, 2);  // first tile computed
      issue(T[s], it + s + NS, std::true_type{});
    }
  }
  NSV_STAMP_AT(a, 3);  // key loop done (wave 0)

  // ---- merge the waves' (max, sum, O) ---------------------------------------
  if (g4 == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      red_m[w][mt * 16 + c] = m_run[mt];
      red_l[w][mt * 16 + c] = l_run[mt];
    }
  }
  const int64_t pbase = ((int64_t)pair * a.S + split) * a.Mv;
  // split partials with the agent-scope cache policy (this split's rows)
  const __amdgpu_buffer_rsrc_t prs = block_rsrc(a.part_o + pbase * DH);
  // ---- in-kernel split merge, per head-dim slice: the nsplit workgroups of
  // a (pair, slice) count in after their partials are acknowledged (each
  // writes its split's (max, sum), identical across slices); the last one
  // combines the splits' partials of its slice, in split order (the result
  // does not depend on which came last), with the ordering protocol of the
  // key-split kernel's merge
  auto merge_splits = [&]() {
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int slot = counter_slot(pair * a.dqc + dq);
    if (tid == 0)
      ds_last = __hip_atomic_fetch_add(&a.counters[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                (unsigned)(nsplit - 1);
    __syncthreads();
    NSV_STAMP_AT(a, 5);  // arrival counted
    if (!uniform(ds_last)) return;
    if (tid == 0) __hip_atomic_store(&a.counters[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int64_t base0 = (int64_t)pair * a.S * a.Mv;  // row 0 of split 0
    const __amdgpu_buffer_rsrc_t ors = block_rsrc(a.part_o + base0 * DH);
    const __amdgpu_buffer_rsrc_t mrs = block_rsrc(a.part_ml + base0 * 2);
    constexpr int C4 = DC / 4;
    constexpr int ITEMS = (MP * C4 + NT - 1) / NT;  // (row, 4 dims of this slice) items per thread
    constexpr int CW = ITEMS <= 2 ? 8 : 4;          // splits whose values one round trip loads
    bool iok[ITEMS];
    unsigned ioff[ITEMS], imlo[ITEMS];
    uint2* idst[ITEMS];
    float M[ITEMS], den[ITEMS];
    f32x4 num[ITEMS];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int qd = tid + j * NT;
      int m = qd / C4;
      const int c4 = qd - m * C4;
      const int g = div_small(m, a.QL), t = m - g * a.QL;
      const bool ok = m < a.Mv && t < qlen;
      iok[j] = ok;
      m = ok ? m : 0;  // (items past the rows load row 0 and are discarded)
      ioff[j] = (unsigned)(m * DH + dq * DC + c4 * 4) * 4u;
      imlo[j] = (unsigned)m * 8u;
      idst[j] = reinterpret_cast<uint2*>((bf16_t*)a.out +
                                         ((int64_t)(q0 + (ok ? t : 0)) * a.H + hk * a.Gs + a.g0 + (ok ? g : 0)) * DH +
                                         dq * DC + c4 * 4);
      M[j] = kNegInf;
      den[j] = 0.f;
      num[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int s0 = 0; s0 < nsplit; s0 += CW) {
      float2 ml[ITEMS][CW];
      f32x4 op[ITEMS][CW];
#pragma unroll
      for (int k = 0; k < CW; ++k) {
        const unsigned rows = (unsigned)(uniform(min(s0 + k, nsplit - 1)) * a.Mv);  // past nsplit: weight 0 below
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
          ml[j][k] = load8_agent(mrs, imlo[j], rows * 8u);
          op[j][k] = load16_agent(ors, ioff[j], rows * (DH * 4u));
        }
      }
#pragma unroll
      for (int j = 0; j < ITEMS; ++j)
#pragma unroll
        for (int k = 0; k < CW; ++k) {
          const float ms = ml[j][k].x + (s0 + k < nsplit ? 0.f : kNegInf);  // stored maxima are finite or -inf
          const float Mn = fmaxf(M[j], ms);
          const float ref = Mn == kNegInf ? 0.f : Mn;
          const float a0 = __builtin_amdgcn_exp2f(M[j] - ref), a1 = __builtin_amdgcn_exp2f(ms - ref);
          den[j] = den[j] * a0 + ml[j][k].y * a1;
          num[j] = num[j] * a0 + op[j][k] * a1;
          M[j] = Mn;
        }
    }
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      if (!iok[j]) continue;
      const float inv = den[j] > 0.f ? 1.f / den[j] : 0.f;
      const uint32_t lo = pack_bf16x2(num[j][0] * inv, num[j][1] * inv);
      const uint32_t hi = pack_bf16x2(num[j][2] * inv, num[j][3] * inv);
      *idst[j] = make_uint2(lo, hi);
    }
    NSV_STAMP_AT(a, 6);  // merge stores issued (last split)
  };
  if constexpr (PARK) {
    // lane (g4, c) element i of tile (dt, mt) is O[16*mt + c][16*dt + 4*g4 + i]
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<f32x4*>(&park[(w * MP + mt * 16 + c) * RSTR + dt * 16 + g4 * 4]) = acc[dt][mt];
    __syncthreads();
    NSV_STAMP_AT(a, 7);  // every wave's key loop done, O parked
    constexpr int C4 = DC / 4;
    for (int qd = tid; qd < a.Mv * C4; qd += NT) {
      const int m = qd / C4, c4 = qd - m * C4;
      float M = kNegInf;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, red_m[ww][m]);
      const float ref = (M == kNegInf) ? 0.f : M;
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
      float L = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        const float f = __builtin_amdgcn_exp2f((red_m[ww][m] - ref) * sc);
        L = fmaf(red_l[ww][m], f, L);
        o += f * *reinterpret_cast<const f32x4*>(&park[(ww * MP + m) * RSTR + c4 * 4]);
      }
      if (nsplit == 1) {
        const int g = div_small(m, a.QL), t = m - g * a.QL;
        if (t >= qlen) continue;
        const float inv = (L > 0.f && row_pos[m] >= 0) ? 1.f / L : 0.f;
        bf16_t* dst = (bf16_t*)a.out + ((int64_t)(q0 + t) * a.H + hk * a.Gs + a.g0 + g) * DH + dq * DC + c4 * 4;
        const uint32_t lo = pack_bf16x2(o[0] * inv, o[1] * inv);
        const uint32_t hi = pack_bf16x2(o[2] * inv, o[3] * inv);
        *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
      } else {
        if (row_pos[m] < 0) o = f32x4{0.f, 0.f, 0.f, 0.f};
        store16_agent(prs, (unsigned)(m * DH + dq * DC + c4 * 4) * 4u, o);
      }
    }
    if (nsplit > 1 && (dq == 0 || a.dmerge) && tid < a.Mv) {
      float M = kNegInf;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, red_m[ww][tid]);
      const float ref = (M == kNegInf) ? 0.f : M;
      float L = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) L += red_l[ww][tid] * __builtin_amdgcn_exp2f((red_m[ww][tid] - ref) * sc);
      store_agent(reinterpret_cast<uint64_t*>(&a.part_ml[(pbase + tid) * 2]),
                  row_pos[tid] >= 0 && M != kNegInf ? M * sc : kNegInf, row_pos[tid] >= 0 ? L : 0.f);
    }
    NSV_STAMP_AT(a, 4);  // waves merged, partials issued
    if (nsplit > 1 && a.dmerge) merge_splits();
    return;
  }
  __syncthreads();  // also: every wave is done with its V staging rows
  if (tid < MP) {
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, red_m[ww][tid]);
    const float ref = (M == kNegInf) ? 0.f : M;
    float L = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) L += red_l[ww][tid] * __builtin_amdgcn_exp2f((red_m[ww][tid] - ref) * sc);
    row_ms[tid] = M == kNegInf ? kNegInf : M * sc;  // partials carry the log2-domain max
    row_l[tid] = L;
  }
  float fac[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + c;
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, red_m[ww][m]);
    fac[mt] = __builtin_amdgcn_exp2f((m_run[mt] - ((M == kNegInf) ? 0.f : M)) * sc);
  }
  float* region = reinterpret_cast<float*>(smem);  // [NW][MTP * 16][RSTR]
  constexpr int C4 = DC / 4;
#pragma unroll
  for (int mp = 0; mp < MT; mp += MTP) {
    if (mp > 0) __syncthreads();  // previous pass fully read
    // lane (g4, c) element i of tile (dt, mt) is O[16*mt + c][16*dt + 4*g4 + i]
#pragma unroll
    for (int mt = mp; mt < mp + MTP && mt < MT; ++mt)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<f32x4*>(&region[(w * MTP * 16 + (mt - mp) * 16 + c) * RSTR + dt * 16 + g4 * 4]) =
            acc[dt][mt] * fac[mt];
    __syncthreads();
    for (int qd = tid; qd < MTP * 16 * C4; qd += NT) {
      const int r = qd / C4, c4 = qd - r * C4;
      const int m = mp * 16 + r;
      if (m >= a.Mv) continue;
      f32x4 o = *reinterpret_cast<const f32x4*>(&region[r * RSTR + c4 * 4]);
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) o += *reinterpret_cast<const f32x4*>(&region[(ww * MTP * 16 + r) * RSTR + c4 * 4]);
      if (nsplit == 1) {
        const int g = div_small(m, a.QL), t = m - g * a.QL;
        if (t >= qlen) continue;
        const float L = row_l[m];
        const float inv = (L > 0.f && row_pos[m] >= 0) ? 1.f / L : 0.f;
        bf16_t* dst = (bf16_t*)a.out + ((int64_t)(q0 + t) * a.H + hk * a.Gs + a.g0 + g) * DH + dq * DC + c4 * 4;
        const uint32_t lo = pack_bf16x2(o[0] * inv, o[1] * inv);
        const uint32_t hi = pack_bf16x2(o[2] * inv, o[3] * inv);
        *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
      } else {
        if (row_pos[m] < 0) o = f32x4{0.f, 0.f, 0.f, 0.f};
        store16_agent(prs, (unsigned)(m * DH + dq * DC + c4 * 4) * 4u, o);
      }
    }
  }
  if (nsplit > 1 && (dq == 0 || a.dmerge) && tid < a.Mv)
    store_agent(reinterpret_cast<uint64_t*>(&a.part_ml[(pbase + tid) * 2]), row_pos[tid] >= 0 ? row_ms[tid] : kNegInf,
                row_pos[tid] >= 0 ? row_l[tid] : 0.f);
  if (nsplit > 1 && a.dmerge) merge_splits();
}

// ---------------------------------------------------------------------------
// bf16 key-split kernel: workgroup = (pair, key split), full head dim.
// ---------------------------------------------------------------------------
// Each workgroup reads only its split's K/V rows, so HBM and every CU see
// each byte once; a pair's context is cut into num_splits() even splits so
// that the grid covers the chip, and the merge kernel combines the splits'
// partials.  (The d-sliced kernel above instead re-reads a pair's K once per
// head-dim slice through L1; at these shapes that re-read, not arithmetic,
// bounds it.)
//
// Waves take interleaved 16-key tiles.  Per tile:
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16, A = K rows straight from HBM
//                 (lane (g4, c): key c, dims 32 ks + 8 g4 .. +7);
//   O^T += V^T P^T  v_mfma_f32_16x16x16_bf16: the S^T accumulator (lane
//                 (g4, c) element i = key 4 g4 + i, query row c) is already
//                 the B operand P^T; V^T comes from the wave's LDS copy of
//                 the tile through one transposing read per 16 dims.
// Each wave keeps one tile in flight: the next is issued when one lands.
// The sequence's whole block-table row is fetched in the first round trip
// (with the context length and query range), so no load waits on another.
#ifndef NSV_KS_WROW
#define NSV_KS_WROW 1
#endif
// WROW: K tiles arrive as whole 2*DH-byte rows (VCH lanes per key, KPI keys
// per load) and are reshaped through a per-wave LDS tile (chunk X of key r
// at slot X ^ (r % VCH)) into the operand layout; a CU ingests whole rows
// several times faster than the operand order's 64 bytes from each of 16
// keys (config 4 on MI355X: 369 -> 356 us per call).
template <int MT, int DH, int NW, bool WROW = (NSV_KS_WROW != 0)>
__global__ __launch_bounds__(NW * 64, 8 / NW) void verify_attn_ks_kernel(VerifyArgs a) {
  constexpr int NT = NW * 64;
  constexpr int TK = 16;          // keys per wave tile
  constexpr int KS = DH / 32;     // k-steps of S^T
  constexpr int DT = DH / 16;     // 16-dim tiles of O^T
  constexpr int MP = MT * 16;     // padded query rows
  constexpr int VCH = DH / 8;     // 16-byte chunks per key row
  constexpr int KPI = NSV_WAVE / VCH;  // keys per coalesced V load
  constexpr int VL = TK / KPI;    // V loads per lane per tile
  constexpr int VSTR = DH + 16;   // staged V row stride (bf16): an odd multiple of 32 bytes
  constexpr int RSTR = DH + 4;    // merge-region row stride (floats)
  constexpr int KSTAGE = WROW ? NW * TK * DH * 2 : 0;  // whole-row K tiles
  constexpr int STAGE = NW * TK * VSTR * 2 + KSTAGE;
  constexpr int MROWS = MP < 32 ? MP : 32;  // query rows one merge pass covers
  constexpr int MPASS = (MP + MROWS - 1) / MROWS;
  constexpr int MERGE_BYTES = NW * MROWS * RSTR * 4;  // every wave's O for MROWS rows
  constexpr int SMEM = STAGE > MERGE_BYTES ? STAGE : MERGE_BYTES;

  // One LDS block, the small arrays first: their addresses then fit the
  // 16-bit offset field of the LDS instructions, so the merge addresses them
  // from one base register instead of computing each address.
  struct __attribute__((aligned(16))) Lds {
    float red_m[NW][MP];
    float red_l[NW][MP];
    float row_l[MP];
    float row_ms[MP];
    int row_pos[MP];
    int is_last;
    int pages[kMaxSplitPages];
    // The workgroup's query rows, the B operand of S^T, shared by the 8 waves
    // (held in registers they would take 4 KS VGPRs per m-tile from the K/V
    // pipeline); chunk X of row m at slot X ^ (m % VCH), so the 16 rows a
    // B-operand read touches fall in distinct banks.
    __attribute__((aligned(16))) unsigned char q_lds[MP * DH * 2];
    __attribute__((aligned(16))) unsigned char smem[SMEM];
  };
  __shared__ Lds lds;
  auto& red_m = lds.red_m;
  auto& red_l = lds.red_l;
  auto& row_l = lds.row_l;
  auto& row_ms = lds.row_ms;
  auto& row_pos = lds.row_pos;
  auto& is_last = lds.is_last;
  auto& pages = lds.pages;
  unsigned char* const q_lds = lds.q_lds;
  unsigned char* const smem = lds.smem;

  // ---- workgroup -> (pair, split): grid (8 P8, splits), so workgroup
  // y * 8 P8 + x runs on XCD x % 8 -- every split of a pair on one XCD
  fetch_args(a);
  NSV_STAMP_AT(a, 0);  // entry
  NSV_STAMP_XCC(a);
  const int pair_raw = blockIdx.x;
  const int split = blockIdx.y;
  // (the grid rounds the pair count up to a multiple of 8: workgroups past
  // the last pair read its metadata and leave once it is back -- an exit
  // before those loads would put the kernel arguments the loads need into a
  // second, dependent round trip)
  const int pair = min(pair_raw, a.npairs - 1);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, c = lane & 15;
  const int b = div_small(pair, a.Hkv), hk = pair - b * a.Hkv;

  // ---- first round trip: block-table row, context length, query range, all
  // issued before any is used (entries past the row read its last one and
  // are not stored)
  const int32_t* btrow = a.block_tables + (int64_t)b * a.max_blocks;
  constexpr int PPT = (kMaxSplitPages + NT - 1) / NT;
  int pv[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) pv[i] = btrow[min(tid + i * NT, a.max_blocks - 1)];
  const int64_t ctx_raw = a.context_lens[b];
  const int q0 = uniform(a.cu_seqlens_q[b]);
  const int q1 = uniform(a.cu_seqlens_q[b + 1]);
  pin_metadata(ctx_raw, q0, q1);
  if (pair_raw >= a.npairs) return;
  const int ctx = clamp_context(a, ctx_raw);
  const int qlen = q1 - q0;
  const int len = split_len_ks(a, ctx);
  const int nsplit = num_splits_ks(ctx, len);
  if (split >= nsplit || qlen < 0) return;  // uniform per workgroup
  const int kb = split * len;
  const int ke = min(ctx, kb + len);
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int j = tid + i * NT;
    if (j < a.max_blocks) pages[j] = pv[i];
  }

  constexpr int QPASS = (MP * VCH + NT - 1) / NT;  // 16-byte query chunks per thread
  u32x4 qt[QPASS];
  int qpos[MT];
  int qmin = 0x7fffffff;
  auto load_q = [&]() {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + c;
      const int g = div_small(m, a.QL), t = m - g * a.QL;
      const bool ok = (m < a.Mv) && (t < qlen);
      qpos[mt] = load_pos(a.positions, ok ? q0 + t : 0);
    }
    // padded and missing rows read the sequence's first row (their scores are masked)
#pragma unroll
    for (int i = 0; i < QPASS; ++i) {
      const int idx = tid + i * NT;
      const int m = idx / VCH, ch = idx % VCH;
      const int g = div_small(m, a.QL), t = m - g * a.QL;
      const bool ok = (idx < MP * VCH) && (m < a.Mv) && (t < qlen);
      const int row = ok ? q0 + t : 0;
      const int gg = ok ? g : 0;
      qt[i] = load16((const bf16_t*)a.q + ((int64_t)row * a.H + hk * a.Gs + a.g0 + gg) * DH + ch * 8);
    }
  };
  auto store_q = [&]() {
#pragma unroll
    for (int i = 0; i < QPASS; ++i) {
      const int idx = tid + i * NT;
      const int m = idx / VCH, ch = idx % VCH;
      if (idx < MP * VCH) *reinterpret_cast<u32x4*>(q_lds + m * (DH * 2) + ((ch ^ (m % VCH)) << 4)) = qt[i];
    }
  };
  auto finish_positions = [&]() {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + c;
      const int g = div_small(m, a.QL), t = m - g * a.QL;
      const bool ok = (m < a.Mv) && (t < qlen);
      qpos[mt] = ok ? qpos[mt] : -1;
      if (qpos[mt] >= 0) qmin = min(qmin, qpos[mt]);
      if (w == 0 && g4 == 0) row_pos[m] = qpos[mt];
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) qmin = min(qmin, __shfl_xor(qmin, o, NSV_WAVE));
    qmin = __builtin_amdgcn_readfirstlane(qmin);
  };

  float m_run[MT], l_run[MT];  // exponent reference (raw-score units; -inf until a finite score), running sum
  f32x4 acc[DT][MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    m_run[mt] = kNegInf;
    l_run[mt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const float sc = a.scale_log2;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const unsigned row_bytes = (unsigned)a.Hkv * DH * 2;  // bytes between consecutive keys of a page
  const size_t page_bytes = (size_t)row_bytes << a.bs_log2;
  const char* kbase = (const char*)a.k_cache + hk * DH * 2;
  const char* vbase = (const char*)a.v_cache + hk * DH * 2;
  uint16_t* vl = reinterpret_cast<uint16_t*>(smem) + w * TK * VSTR;
  unsigned char* kl = smem + NW * TK * VSTR * 2 + (WROW ? w * TK * DH * 2 : 0);
  __syncthreads();  // block-table row visible
  NSV_STAMP_AT(a, 1);  // metadata back

  const int ntiles = (ke - kb + TK - 1) / TK;
  const int niter = (ntiles + NW - 1) / NW;  // same trip count in every wave

  struct Tile {
    u32x4 k[KS];  // K as the A operand of S^T, or (WROW) whole rows like v
    u32x4 v[VL];  // V rows, coalesced: load j, lane -> (key j * KPI + lane / VCH, chunk lane % VCH)
    int n0;
    int nvalid;   // the tile's existing keys are exactly its first nvalid
  };

  // Issue every load of wave-tile `it` (tiles never cross a page: splits
  // start on 16-key boundaries and pages hold a power of two >= 16 keys).
  // Missing keys read a row that exists.  A wave's first tile is always
  // issued (a tile past the split reads the pool's first row), so the
  // compiler's wait for the query rows staged before the first barrier
  // stays exact and that barrier does not wait for the tile; a later tile
  // without any key issues no load (the loop waits for vmcnt(0) anyway),
  // so no dummy loads queue in the CU's address unit beside real tiles.
  auto issue = [&](Tile& T, int it, auto skip_empty) {
    T.n0 = kb + (it * NW + w) * TK;
    int nvalid = min(max(ke - T.n0, 0), TK);
    int pg = nvalid > 0 ? pages[T.n0 >> a.bs_log2] : -1;
    pg = __builtin_amdgcn_readfirstlane(pg);
    if (pg < 0) nvalid = 0;
    T.nvalid = nvalid;
    if constexpr (decltype(skip_empty)::value) {
      if (nvalid == 0) return;  // uniform
    }
    const size_t page_off = (size_t)(pg < 0 ? 0 : pg) * page_bytes;
    const char* kp = kbase + page_off;
    const char* vp = vbase + page_off;
    const unsigned base_key = (unsigned)(T.n0 & bs_mask);
    if constexpr (WROW) {
#pragma unroll
      for (int j = 0; j < KS; ++j) {  // 16 keys x VCH chunks = KS loads of 64 chunks
        const int r = j * KPI + lane / VCH, ch = lane % VCH;
        T.k[j] = load16_stream(kp + (base_key + (r < nvalid ? r : 0)) * row_bytes + ch * 16);
      }
    } else {
      const unsigned off = (base_key + (c < nvalid ? c : 0)) * row_bytes + g4 * 16;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) T.k[ks] = load16_stream(kp + off + ks * 64);
    }
#pragma unroll
    for (int j = 0; j < VL; ++j) {
      const int r = j * KPI + lane / VCH, ch = lane % VCH;
      const unsigned off = (base_key + (r < nvalid ? r : 0)) * row_bytes + ch * 16;
      T.v[j] = load16_stream(vp + off);
    }
  };

  auto compute = [&](const Tile& T) {
    if (T.nvalid == 0) return;  // uniform: nothing of this tile exists
    u32x4 kA[KS];
    if constexpr (WROW) {
      // row-order tile -> LDS (this wave's rows; its LDS ops complete in order) -> operand order:
      // lane (g4, c) takes key c, chunk 4 ks + g4
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const int r = j * KPI + lane / VCH, ch = lane % VCH;
        *reinterpret_cast<u32x4*>(kl + r * (DH * 2) + ((ch ^ (r % VCH)) << 4)) = T.k[j];
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kA[ks] = *reinterpret_cast<const u32x4*>(kl + c * (DH * 2) + (((ks * 4 + g4) ^ (c % VCH)) << 4));
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kA[ks] = T.k[ks];
    }
    f32x4 sacc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        sv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(kA[ks]),
            as_bf16x8(*reinterpret_cast<const u32x4*>(q_lds + (mt * 16 + c) * (DH * 2) + (((ks * 4 + g4) ^ (c % VCH)) << 4))),
            sv, 0, 0, 0);
      sacc[mt] = sv;
    }
    // stage V (this wave's private LDS rows; a wave's LDS ops complete in order)
#pragma unroll
    for (int j = 0; j < VL; ++j) {
      const int r = j * KPI + lane / VCH, ch = lane % VCH;
      *reinterpret_cast<u32x4*>(vl + r * VSTR + ch * 8) = T.v[j];
    }
    // missing keys and keys past a row's position get -inf (exact 0 weight)
    const bool full = (T.nvalid == TK) && (T.n0 + TK - 1 <= qmin);
    if (!full) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = g4 * 4 + i;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          sacc[mt][i] = (r < T.nvalid && T.n0 + r <= qpos[mt]) ? sacc[mt][i] : kNegInf;
      }
    }
    // Online softmax with a lazily moved reference point: a row's weights are
    // exp2((s - m_ref) sc), and m_ref follows the row's running maximum only
    // when that maximum passes it by more than kRefSlack in the log2 domain,
    // so a weight stays <= 2^kRefSlack and the accumulators are rescaled on
    // those tiles alone (a row's first finite scores set it; its
    // accumulators are still zero then).  The weights are a constant factor
    // times the ones a reference at the running maximum would give, and their
    // bf16 rounding is relative, so the result is the same softmax.
    i16x4 pB[MT];
    float alpha[MT];
    bool moved = false;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float mx = __builtin_fmaxf(__builtin_fmaxf(sacc[mt][0], sacc[mt][1]), __builtin_fmaxf(sacc[mt][2], sacc[mt][3]));
      mx = row_max4(mx);
      const float m_old = m_run[mt];
      const float m_new = fmaxf(m_old, mx);
      // (m_old -inf and m_new finite: +inf, a move; both -inf: NaN, none)
      const bool shift = (m_new - m_old) * sc > kRefSlack;
      const float m_ref = shift ? m_new : m_old;
      alpha[mt] = shift ? __builtin_amdgcn_exp2f((m_old - m_new) * sc) : 1.f;
      moved |= shift && m_old != kNegInf;
      const float nb = (m_ref == kNegInf) ? 0.f : -m_ref * sc;  // exp2 bias
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(sacc[mt][i], sc, nb));
      l_run[mt] = fmaf(l_run[mt], alpha[mt], row_sum4((p[0] + p[1]) + (p[2] + p[3])));
      m_run[mt] = m_ref;
      // P^T as the B operand, rounded to bf16 like the reference's p.to(v.dtype)
      pB[mt] = __builtin_bit_cast(i16x4, make_uint2(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])));
    }
    if (__ballot(moved)) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt][mt] *= alpha[mt];
    }
    __builtin_amdgcn_wave_barrier();
    // O^T += V^T P^T: lane (g4, c) reads V[4 g4 + j][16 dt + c], j = 0..3
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint2 vt = lds_read_tr(vl + (g4 * 4 + (c >> 2)) * VSTR + dt * 16 + (c & 3) * 4);
      const i16x4 vA = __builtin_bit_cast(i16x4, vt);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[dt][mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vA, pB[mt], acc[dt][mt], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- pipeline over this wave's tiles: one tile in flight per wave, the
  // next issued as soon as the current one has landed and before it is
  // computed, so the arithmetic hides under the next tile's flight.  More
  // tiles in flight only queue more requests and lower the memory system's
  // rate for this access pattern (MI355X, graph-replayed: config 2 15.6 us
  // with one, 17.8 with two, 18.2 with every tile of the wave at once;
  // config 4 328.6 us with one against 337.3 with a two-stage pipeline).
  load_q();
  Tile T0, T1;
  __builtin_amdgcn_sched_barrier(0);
  issue(T0, 0, std::false_type{});
  __builtin_amdgcn_sched_barrier(0);
  finish_positions();
  store_q();
  lds_barrier();  // query rows visible; the first tile stays in flight
  for (int it = 0; it < niter; it += 2) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): tile it landed
    __builtin_amdgcn_sched_barrier(0);
    if (it == 0) NSV_STAMP_AT(a, 2);  // first tile landed
    if (it + 1 < niter) issue(T1, it + 1, std::true_type{});
    __builtin_amdgcn_sched_barrier(0);
    compute(T0);
    if (it + 1 >= niter) break;
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): tile it + 1 landed
    __builtin_amdgcn_sched_barrier(0);
    if (it + 2 < niter) issue(T0, it + 2, std::true_type{});
    __builtin_amdgcn_sched_barrier(0);
    compute(T1);
  }

  NSV_STAMP_AT(a, 3);  // key loop done (wave 0)

  // ---- merge the waves' (max, sum, O) ---------------------------------------
  if (g4 == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      red_m[w][mt * 16 + c] = m_run[mt];
      red_l[w][mt * 16 + c] = l_run[mt];
    }
  }
  __syncthreads();  // also: every wave is done with its staging rows
  NSV_STAMP_AT(a, 7);  // every wave's key loop done
  // every lane: the split's max over the waves for its rows, and its own
  // waves' rescale factor; wave 0 keeps the split's (max, sum) per row
  // (every LDS read of a step is issued before the first is used: the
  // scheduler would otherwise chain them a few at a time)
  float fac[MT];
  float rm[MT][NW], rl[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      rm[mt][ww] = red_m[ww][mt * 16 + c];
      rl[mt][ww] = red_l[ww][mt * 16 + c];  // (used by wave 0; read by all: no branch per read)
    }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + c;
    float M = kNegInf;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, rm[mt][ww]);
    const float ref = (M == kNegInf) ? 0.f : M;
    fac[mt] = __builtin_amdgcn_exp2f((m_run[mt] - ref) * sc);
    if (w == 0 && g4 == 0) {
      float L = 0.f;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) L = fmaf(rl[mt][ww], __builtin_amdgcn_exp2f((rm[mt][ww] - ref) * sc), L);
      const float ms = M == kNegInf ? kNegInf : M * sc;  // partials carry the log2-domain max
      row_ms[m] = ms;
      row_l[m] = L;
    }
  }
  // Every wave's scaled O rows (real rows only: rows >= Mv are padding) go
  // to LDS, MROWS rows per pass (one pass up to 32 rows); then thread tid
  // sums the waves for items (row, 4 dims) tid, tid + NT, ... of the pass.
  // The items a thread sums (ITEMS per pass) are the ones it merges across
  // splits below, so its own split's sums stay in registers.
  float* region = reinterpret_cast<float*>(smem);  // [NW][MROWS][RSTR]
  constexpr int C4 = DH / 4;
  constexpr int ITEMS = (MROWS * C4 + NT - 1) / NT;
  f32x4 own[MPASS][ITEMS];
  const int64_t pbase = ((int64_t)pair * a.S + split) * a.Mv;
  const __amdgpu_buffer_rsrc_t prs = block_rsrc(a.part_o + pbase * DH);  // this split's partial rows
#pragma unroll
  for (int ps = 0; ps < MPASS; ++ps) {
    if (ps > 0) __syncthreads();  // the previous pass fully read
#pragma unroll
    for (int mt = ps * (MROWS / 16); mt < MT && mt < (ps + 1) * (MROWS / 16); ++mt) {
      const int m = mt * 16 + c;
      if (m < a.Mv) {
        // lane (g4, c) element i of tile (dt, mt) is O[16 mt + c][16 dt + 4 g4 + i]
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          *reinterpret_cast<f32x4*>(&region[(w * MROWS + (m - ps * MROWS)) * RSTR + dt * 16 + g4 * 4]) =
              acc[dt][mt] * fac[mt];
      }
    }
    __syncthreads();
    if (ps == 0) NSV_STAMP_AT(a, 8);  // O rows in LDS
    f32x4 wv[ITEMS][NW];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int r = min((tid + j * NT) / C4, MROWS - 1), c4 = (tid + j * NT) % C4;  // rows past MROWS: discarded
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) wv[j][ww] = *reinterpret_cast<const f32x4*>(&region[(ww * MROWS + r) * RSTR + c4 * 4]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int qd = tid + j * NT;
      const int r = qd / C4, c4 = qd % C4;
      const int m = ps * MROWS + r;
      own[ps][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (r >= MROWS || m >= a.Mv) continue;
      f32x4 o = wv[j][0];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) o += wv[j][ww];
      if (row_pos[m] < 0) o = f32x4{0.f, 0.f, 0.f, 0.f};
      own[ps][j] = o;
      if (nsplit == 1) {
        const int g = div_small(m, a.QL), t = m - g * a.QL;
        if (t >= qlen) continue;
        const float L = row_l[m];
        const float inv = L > 0.f ? 1.f / L : 0.f;
        bf16_t* dst = (bf16_t*)a.out + ((int64_t)(q0 + t) * a.H + hk * a.Gs + a.g0 + g) * DH + c4 * 4;
        const uint32_t lo = pack_bf16x2(o[0] * inv, o[1] * inv);
        const uint32_t hi = pack_bf16x2(o[2] * inv, o[3] * inv);
        *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
      } else {
        store16_agent(prs, (unsigned)(m * DH + c4 * 4) * 4u, o);
      }
    }
  }
  NSV_STAMP_AT(a, 4);  // waves merged, partials issued
  if (nsplit == 1) return;
  // the split's (max, sum) per row, written by wave 0 before the barrier above
  // (stored only now, so that barrier did not wait for the store's acknowledgement)
  if (tid < a.Mv) {
    const bool real = row_pos[tid] >= 0;
    store_agent(reinterpret_cast<uint64_t*>(&a.part_ml[(pbase + tid) * 2]), real ? row_ms[tid] : kNegInf,
                real ? row_l[tid] : 0.f);
  }
  // What the merge needs of this thread's items that no other split holds
  // (validity, offsets, destination, this split's (max, sum)), computed while
  // the stores above are acknowledged and the arrival atomic is in flight:
  // the last split's merge is a chain of single-wave instructions, so every
  // instruction taken off it shortens the kernel.
  bool iok[MPASS][ITEMS];
  unsigned ioff[MPASS][ITEMS], imlo[MPASS][ITEMS];  // byte offsets in a split's partial rows / (max, sum) pairs
  float ims[MPASS][ITEMS], ils[MPASS][ITEMS];
  uint2* idst[MPASS][ITEMS];
#pragma unroll
  for (int ps = 0; ps < MPASS; ++ps)
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int qd = tid + j * NT;
      const int r = qd / C4, c4 = qd % C4;
      int m = ps * MROWS + r;
      const int g = div_small(m, a.QL), t = m - g * a.QL;
      const bool ok = r < MROWS && m < a.Mv && t < qlen;
      iok[ps][j] = ok;
      m = ok ? m : 0;
      ioff[ps][j] = (unsigned)(m * DH + c4 * 4) * 4u;
      imlo[ps][j] = (unsigned)m * 8u;
      const bool real = row_pos[m] >= 0;
      ims[ps][j] = real ? row_ms[m] : kNegInf;
      ils[ps][j] = real ? row_l[m] : 0.f;
      idst[ps][j] = reinterpret_cast<uint2*>(
          (bf16_t*)a.out + ((int64_t)(q0 + (ok ? t : 0)) * a.H + hk * a.Gs + a.g0 + (ok ? g : 0)) * DH + c4 * 4);
    }

  // ---- cross-split merge by the pair's last split to finish ------------------
  // Ordering without release/acquire (which on gfx950 would write back and
  // invalidate whole L2s: 45 us per call measured): the partials above and
  // the (max, sum) pairs are stored with sc1 (agent scope: written through to
  // the device's point of coherence).  Every thread waits for
  // their acknowledgement (vmcnt(0)) before the barrier that precedes the
  // arrival atomic; the split that counts last issues its sc1 loads (served
  // from the point of coherence, past any cached copy) only after
  // the counter's value came back, so it reads every other split's partials.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0)
    is_last = __hip_atomic_fetch_add(&a.counters[counter_slot(pair)], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (unsigned)(nsplit - 1);
  __syncthreads();
  NSV_STAMP_AT(a, 5);  // arrival counted
  if (!uniform(is_last)) return;
  if (tid == 0) __hip_atomic_store(&a.counters[counter_slot(pair)], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int64_t base0 = (int64_t)pair * a.S * a.Mv;  // row 0 of split 0
  const __amdgpu_buffer_rsrc_t ors = block_rsrc(a.part_o + base0 * DH);   // the pair's partial rows
  const __amdgpu_buffer_rsrc_t mrs = block_rsrc(a.part_ml + base0 * 2);   // and (max, sum) pairs
  constexpr int CH = 4;  // beyond 8 splits: splits whose values one round trip loads
  // Splits combine in a fixed order (0, 1, ...), whichever split merges, so
  // the result does not depend on which split finished last.  A row with no
  // key so far (max -inf) takes reference 0, so its weights are exactly 0.
  auto fold = [&](float& M, float& den, f32x4& num, float ms, float ls, f32x4 os) {
    const float Mn = fmaxf(M, ms);
    const float ref = Mn == kNegInf ? 0.f : Mn;
    const float a0 = __builtin_amdgcn_exp2f(M - ref), a1 = __builtin_amdgcn_exp2f(ms - ref);
    den = den * a0 + ls * a1;
    num = num * a0 + os * a1;
    M = Mn;
  };
  auto emit = [&](uint2* dst, float den, f32x4 num) {
    const float inv = den > 0.f ? 1.f / den : 0.f;
    const uint32_t lo = pack_bf16x2(num[0] * inv, num[1] * inv);
    const uint32_t hi = pack_bf16x2(num[2] * inv, num[3] * inv);
    *dst = make_uint2(lo, hi);
  };
  // a real split other than this one (its values are loaded and not used)
  auto other = [&](int sp) { return uniform((sp < nsplit && sp != split) ? sp : (split == 0 ? 1 : 0)); };
  // Up to 8 splits: every value this thread merges, for all its items, in
  // one round trip (items past the rows load row 0 and are discarded).
  // This split's own values are loaded too (they were acknowledged before
  // the arrival), and splits past nsplit load split 0 and weigh 0: every
  // loaded value is used on every path, so the compiler neither moves a load
  // under a branch nor branches on which split is which.
  auto merge_in_one_trip = [&](auto width) {
    constexpr int CW = decltype(width)::value;
    float2 ml[MPASS][ITEMS][CW];
    f32x4 op[MPASS][ITEMS][CW];
#pragma unroll
    for (int k = 0; k < CW; ++k) {
      const unsigned rows = (unsigned)(uniform(k < nsplit ? k : 0) * a.Mv);
#pragma unroll
      for (int ps = 0; ps < MPASS; ++ps)
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
          ml[ps][j][k] = load8_agent(mrs, imlo[ps][j], rows * 8u);
          op[ps][j][k] = load16_agent(ors, ioff[ps][j], rows * (DH * 4u));
        }
    }
    // every item is combined before the first output store: on gfx9 one
    // counter tracks loads and stores, so a load waited for after a store
    // would also wait for the store's acknowledgement.  (One maximum over
    // the splits, then one weight per split: splits past nsplit weigh 0,
    // this split's own values come from registers.)
    float dens[MPASS][ITEMS];
    f32x4 nums[MPASS][ITEMS];
#pragma unroll
    for (int ps = 0; ps < MPASS; ++ps)
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        float ms[CW];
        float M = kNegInf;
#pragma unroll
        for (int k = 0; k < CW; ++k) {
          // (a split past nsplit: its max moved to -inf, so its weight is 0;
          // every stored max is finite or -inf)
          ms[k] = ml[ps][j][k].x + (k < nsplit ? 0.f : kNegInf);
          M = fmaxf(M, ms[k]);
        }
        const float ref = M == kNegInf ? 0.f : M;
        float den = 0.f;
        f32x4 num = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < CW; ++k) {
          const float wk = __builtin_amdgcn_exp2f(ms[k] - ref);  // -inf: 0
          den = fmaf(ml[ps][j][k].y, wk, den);
          num += op[ps][j][k] * wk;
        }
        dens[ps][j] = den;
        nums[ps][j] = num;
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ps = 0; ps < MPASS; ++ps)
#pragma unroll
      for (int j = 0; j < ITEMS; ++j)
        if (iok[ps][j]) emit(idst[ps][j], dens[ps][j], nums[ps][j]);
  };
  if (nsplit <= 4) {
    merge_in_one_trip(std::integral_constant<int, 4>{});
    NSV_STAMP_AT(a, 6);  // merge stores issued (last split)
    return;
  }
  if (nsplit <= 8) {
    merge_in_one_trip(std::integral_constant<int, 8>{});
    NSV_STAMP_AT(a, 6);
    return;
  }
  // more splits: CH per round trip
#pragma unroll
  for (int ps = 0; ps < MPASS; ++ps) {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      if (!iok[ps][j]) continue;
      float M = kNegInf, den = 0.f;
      f32x4 num = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < nsplit; s0 += CH) {
        float2 ml[CH];
        f32x4 op[CH];
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          const unsigned rows = (unsigned)(other(s0 + k) * a.Mv);
          ml[k] = load8_agent(mrs, imlo[ps][j], rows * 8u);
          op[k] = load16_agent(ors, ioff[ps][j], rows * (DH * 4u));
        }
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          const int sp = s0 + k;
          if (sp >= nsplit) break;
          if (sp == split) fold(M, den, num, ims[ps][j], ils[ps][j], own[ps][j]);
          else fold(M, den, num, ml[k].x, ml[k].y, op[k]);
        }
      }
      emit(idst[ps][j], den, num);
    }
  }
}

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

  int split, pair;
  decode_block(a, split, pair);
  if (pair >= a.npairs) return;
  const int lane = threadIdx.x;
  const int b = pair / a.Hkv, hk = pair - b * a.Hkv;
  const int ctx = context_len(a, b);
  const int nsplit = num_splits(a, ctx);
  if (split >= nsplit) return;
  const int tok_begin = split * a.split_tokens;
  const int tok_end = min(ctx, tok_begin + a.split_tokens);
  const int q0 = uniform(a.cu_seqlens_q[b]);
  const int qlen = uniform(a.cu_seqlens_q[b + 1]) - q0;

  // local row r serves query row m = m_base + r of the pair's Mv rows
  for (int idx = lane; idx < MP * DH; idx += NSV_WAVE) {
    const int r = idx / DH, d = idx - r * DH;
    const int m = a.m_base + r;
    const int g = m / a.QL, t = m - g * a.QL;
    const bool ok = (m < a.Mv) && (t < qlen);
    q_s[r][d] = ok ? ((const float*)a.q)[((int64_t)(q0 + t) * a.H + hk * a.Gs + a.g0 + g) * DH + d] : 0.f;
  }
  if (lane < MP) {
    const int m = a.m_base + lane;
    const int g = m / a.QL, t = m - g * a.QL;
    const bool ok = (m < a.Mv) && (t < qlen);
    pos_s[lane] = ok ? load_pos(a.positions, q0 + t) : -1;
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
    for (int r = 0; r < MP; ++r) {
      const int m = a.m_base + r;
      const int g = m / a.QL, t = m - g * a.QL;
      if (m >= a.Mv || t >= qlen) continue;
#pragma unroll
      for (int e = 0; e < E; ++e)
        out[((int64_t)(q0 + t) * a.H + hk * a.Gs + a.g0 + g) * DH + lane + 64 * e] =
            l_run[r] > 0.f ? acc[r][e] / l_run[r] : 0.f;
    }
    return;
  }
  const int64_t base = ((int64_t)pair * a.S + split) * a.Mv + a.m_base;
#pragma unroll
  for (int r = 0; r < MP; ++r) {
    if (a.m_base + r >= a.Mv) continue;
#pragma unroll
    for (int e = 0; e < E; ++e) a.part_o[(base + r) * DH + lane + 64 * e] = acc[r][e];
    if (lane == 0) {
      a.part_ml[(base + r) * 2 + 0] = m_run[r];
      a.part_ml[(base + r) * 2 + 1] = l_run[r];
    }
  }
}

// ---------------------------------------------------------------------------
// Split merge: one workgroup per (pair, 4 query rows of the group), 64 lanes
// per row, D/64 head dims per lane.  Each lane loads its row's (max, sum)
// and its dims of every split's partial together, 8 splits per round trip,
// and folds them with a running max:
//   out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s.
// ---------------------------------------------------------------------------
template <typename OutT, int E>
__global__ __launch_bounds__(256) void verify_merge_kernel(VerifyArgs a) {
  constexpr int DH = 64 * E;
  constexpr int CH = 8;  // splits per round trip
  fetch_args(a);
  const int pair = min((int)blockIdx.x, a.npairs - 1);
  const int m_raw = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int m = min(m_raw, a.Mv - 1);
  const int lane = threadIdx.x & 63;
  const int b = pair / a.Hkv, hk = pair - b * a.Hkv;
  const int64_t base = (int64_t)pair * a.S * a.Mv + m;  // row of split 0
  // The first CH splits' values are loaded with the metadata, in one round
  // trip (exits only after every load was issued; splits past the plan's S
  // read split 0).  Splits the sequence does not have hold stale values,
  // possibly not finite: they are masked off bitwise, not multiplied by a
  // zero weight.
  float2 ml0[CH];
  float os0[CH][E];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int64_t r = base + (int64_t)(j < a.S ? j : 0) * a.Mv;
    ml0[j] = *reinterpret_cast<const float2*>(&a.part_ml[r * 2]);
#pragma unroll
    for (int e = 0; e < E; ++e) os0[j][e] = a.part_o[r * DH + e * 64 + lane];
  }
  const int64_t ctx_raw = a.context_lens[b];
  const int q0 = uniform(a.cu_seqlens_q[b]);
  const int q1 = uniform(a.cu_seqlens_q[b + 1]);
  pin_metadata(ctx_raw, q0, q1);
  if ((int)blockIdx.x >= a.npairs || m_raw >= a.Mv) return;
  const int ctx = clamp_context(a, ctx_raw);
  const int nsplit = num_splits(a, ctx);
  if (nsplit <= 1) return;  // written by the attention kernel itself
  const int qlen = q1 - q0;
  const int g = m / a.QL, t = m - g * a.QL;
  if (t >= qlen) return;
  auto keep = [](float v, uint32_t mask, uint32_t other) { return __uint_as_float((__float_as_uint(v) & mask) | (other & ~mask)); };
  float M = kNegInf, den = 0.f, num[E];
#pragma unroll
  for (int e = 0; e < E; ++e) num[e] = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += CH) {
    float ms[CH], ls[CH], os[CH][E];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      float2 ml;
      float o[E];
      if (s0 == 0) {
        ml = ml0[j];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = os0[j][e];
      } else {
        const int sp = s0 + j < nsplit ? s0 + j : s0;
        const int64_t r = base + (int64_t)sp * a.Mv;
        ml = *reinterpret_cast<const float2*>(&a.part_ml[r * 2]);
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = a.part_o[r * DH + e * 64 + lane];
      }
      const uint32_t mask = s0 + j < nsplit ? 0xffffffffu : 0u;  // absent split: max -inf, sum 0, values 0
      ms[j] = keep(ml.x, mask, 0xff800000u);
      ls[j] = keep(ml.y, mask, 0u);
#pragma unroll
      for (int e = 0; e < E; ++e) os[j][e] = keep(o[e], mask, 0u);
    }
    float Mn = M;
#pragma unroll
    for (int j = 0; j < CH; ++j) Mn = fmaxf(Mn, ms[j]);
    if (Mn == kNegInf) continue;  // no key of this row so far
    const float r = exp2f(M - Mn);  // M = -inf: 0 (nothing accumulated yet)
    den *= r;
#pragma unroll
    for (int e = 0; e < E; ++e) num[e] *= r;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const float wgt = exp2f(ms[j] - Mn);  // -inf (absent split or no key): 0
      den = fmaf(wgt, ls[j], den);
#pragma unroll
      for (int e = 0; e < E; ++e) num[e] = fmaf(wgt, os[j][e], num[e]);
    }
    M = Mn;
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  OutT* dst = (OutT*)a.out + ((int64_t)(q0 + t) * a.H + hk * a.Gs + a.g0 + g) * DH;
#pragma unroll
  for (int e = 0; e < E; ++e) dst[e * 64 + lane] = (OutT)(num[e] * inv);
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
  int G, QL, Mv, MT, split, S, dqc;
  int Gs;         // query heads per kv head; launches serve G of them at a time (Gs / G launches)
  int ks;         // 1: key-split kernel, 0: d-sliced kernel (bf16)
  int ks_splits;  // key-split kernel, automatic splits per sequence (split == 0)
};

int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

// Compute units of the current device (256 on MI355X); the plan only uses
// it to size the grid, so a failed query falls back to that figure.
int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  return cus;
}

int make_plan(int B, int H, int Hkv, int D, int block_size, int max_blocks, int max_q_len, int dtype,
              int kv_split_tokens, int cus, Plan* p) {
  if (B < 0 || H <= 0 || Hkv <= 0 || max_blocks <= 0 || max_q_len <= 0) return NSV_ERR_ARG;
  if (dtype != NSV_F32 && dtype != NSV_BF16) return NSV_ERR_ARG;
  if (H % Hkv) return NSV_ERR_UNSUPPORTED;
  if (D != 64 && D != 128) return NSV_ERR_UNSUPPORTED;
  if (ilog2_exact(block_size) < 0) return NSV_ERR_UNSUPPORTED;
  // The kernels hold at most 64 query rows (group heads x query tokens) per
  // (sequence, kv head); a larger group is served G heads at a time, G the
  // largest divisor of the group whose rows fit, one launch (and merge) per
  // head subset.  Each subset re-reads the pair's K/V.
  if (max_q_len > 64) return NSV_ERR_UNSUPPORTED;
  p->Gs = H / Hkv;
  p->G = p->Gs;
  while (p->G * max_q_len > 64) {
    int g = p->G - 1;
    while (p->Gs % g) --g;
    p->G = g;
  }
  p->QL = max_q_len;
  p->Mv = p->G * max_q_len;
  p->MT = (p->Mv + 15) / 16;
  const int64_t max_ctx = (int64_t)max_blocks * block_size;
  if (max_ctx > (int64_t)1 << 30) return NSV_ERR_UNSUPPORTED;
  if (kv_split_tokens < 0 || (kv_split_tokens % 128)) return NSV_ERR_ARG;
  const int64_t pairs = (int64_t)B * Hkv;
  // longest split whose block-table slice fits the kernel's LDS copy
  const int64_t page_cap = ((int64_t)(kMaxSplitPages - 1) * block_size) / 128 * 128;
  int64_t split = kv_split_tokens;
  p->dqc = 1;
  p->ks = 0;
  p->ks_splits = 0;
  // Kernel choice (bf16).  The key-split kernel reads every K/V byte once
  // per CU but pays about three memory round trips to merge a pair's splits;
  // the d-sliced kernel needs no cross-workgroup merge but re-reads the
  // pair's K through every slice's L1, whose fill rate (~25 GB/s per CU)
  // then bounds it.  Measured on MI355X (Qwen3-0.6B layer, ~1.25k keys,
  // graph-replayed over 28 pools; d-sliced with its merge launch against
  // the best key split): 8 pairs 11.1 against 11.5 us, 16 pairs 12.7
  // against 12.0, 32 pairs 14.4 (d-sliced: 16.2) against 13.3, 64 pairs
  // 17.2 against 16.8; at 128 pairs x 16k-32k keys the key-split kernel is
  // 2x faster.  So key-split from a sixteenth as many pairs as resident
  // workgroups, or when a table holds >= 4096 keys, or for one 16-row tile
  // of query rows (decode-shaped calls: at 8 pairs x 1.25k keys and 2 or 4
  // rows per pair, 8.0 us against 9.4 for the d-sliced kernel and its merge
  // launch; with its in-kernel merge and query staging the d-sliced kernel
  // there still made a self-drafting b1 round 7.30 -> 7.38 ms).
  const int64_t ks_slots = (int64_t)cus * (8 / kKsWaves);  // resident workgroups
  // (contexts under 2^22 keys: the kernel's split arithmetic, div_small)
  const bool ks_fits = p->MT <= 3 && block_size >= 16 && max_blocks <= kMaxSplitPages && max_ctx < (1 << 22) &&
                       (pairs <= kMaxCounterPairs || (kv_split_tokens == 0 && pairs >= ks_slots));
  const bool ks_wins = kv_split_tokens > 0 || pairs * 16 >= ks_slots || max_ctx >= 4096 || p->MT == 1;
  if (dtype == NSV_BF16 && ks_fits && ks_wins) {
    // key-split kernel: each sequence's keys evenly over about CUs / pairs
    // splits (none when the pairs alone cover the chip), but no split
    // shorter than 160 keys (shorter splits pay the merge for too few loads:
    // at 8 pairs x 1.25k keys, 8 splits take 11.5 us, 10 12.7, 16 12.7; at
    // 32 pairs 8 take 13.3 against 14.4 for 5), or the caller's fixed split
    // length
    p->ks = 1;
    if (split == 0) {
      int64_t S = pairs > 0 ? (ks_slots + pairs / 2) / pairs : 1;
      // (merges of more than 8 splits take more than one round trip: those
      // splits are at least 512 keys long)
      int64_t max_splits = (max_ctx + 159) / 160;
      if (max_splits > 8) max_splits = std::max<int64_t>(8, (max_ctx + 511) / 512);
      if (S > max_splits) S = max_splits;
      if (S > 64) S = 64;
      if (S < 1 || pairs > kMaxCounterPairs) S = 1;
      p->ks_splits = (int)S;
      p->split = 0;
      p->S = (int)S;
    } else {
      p->split = (int)split;
      p->S = (int)((max_ctx + split - 1) / split);
    }
    if (p->S > 8192) return NSV_ERR_UNSUPPORTED;  // the merge stages 2 * S floats in LDS
    return NSV_OK;
  }
  if (dtype == NSV_BF16) {
    // widest head-dim slice whose double-buffered K/V tiles and accumulators
    // fit the register file without spilling: 64 dims up to 32 padded query
    // rows, 32 beyond
    const int dc_max = p->MT <= 2 ? 64 : 32;
    p->dqc = D > dc_max ? D / dc_max : 1;
    while (pairs * p->dqc < cus && p->dqc < D / 32) p->dqc *= 2;
    if (split == 0) {
      split = (max_ctx + 127) / 128 * 128;  // one split per sequence ...
      const int64_t units = pairs * p->dqc;
      if (units > 0 && units < cus) {        // ... unless the grid would leave CUs idle
        const int64_t want = (cus + units - 1) / units;
        split = ((max_ctx + want - 1) / want + 127) / 128 * 128;
      }
      if (split > page_cap) split = page_cap;
      if (split < 128) split = 128;
    } else if (split > page_cap) {
      return NSV_ERR_UNSUPPORTED;
    }
  } else if (split == 0) {
    // fp32: enough one-wave workgroups to cover the chip a few times over
    split = 256;
    while (pairs * ((max_ctx + split - 1) / split) > 1024 && split < 8192) split *= 2;
  }
  p->split = (int)split;
  p->S = (int)((max_ctx + split - 1) / split);
  if (p->S > 8192) return NSV_ERR_UNSUPPORTED;  // the merge stages 2 * S floats in LDS
  return NSV_OK;
}

// Workspace: [per-pair counters, 256-byte aligned][part_ml, 256-byte aligned][part_o].
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t counter_bytes(int, int) { return (size_t)kMaxCounterPairs * sizeof(unsigned); }

size_t ml_bytes(int B, int Hkv, const Plan& p) { return align256((size_t)B * Hkv * p.S * p.Mv * 2 * sizeof(float)); }

size_t workspace_bytes_for(int B, int Hkv, int D, const Plan& p) {
  if (p.S <= 1) return 0;
  return counter_bytes(B, Hkv) + ml_bytes(B, Hkv, p) + (size_t)B * Hkv * p.S * p.Mv * (size_t)D * sizeof(float);
}

template <int MT, int DH, int DC>
void launch_bf16_dc(const VerifyArgs& a, dim3 grid, hipStream_t s) {
  if (a.bs_log2 >= 5)
    hipLaunchKernelGGL((verify_attn_bf16_kernel<MT, DH, DC, true, bf16_stages(MT, DH, DC, true)>), grid, dim3(kBf16Waves * 64), 0, s, a);
  else
    hipLaunchKernelGGL((verify_attn_bf16_kernel<MT, DH, DC, false, bf16_stages(MT, DH, DC, false)>), grid, dim3(kBf16Waves * 64), 0, s, a);
}

template <int MT>
int launch_ks(const VerifyArgs& a, int D, dim3 grid, hipStream_t s) {
  if constexpr (MT <= 3) {
    constexpr int NW = kKsWaves;
    if (D == 128)
      hipLaunchKernelGGL((verify_attn_ks_kernel<MT, 128, NW>), grid, dim3(NW * 64), 0, s, a);
    else
      hipLaunchKernelGGL((verify_attn_ks_kernel<MT, 64, NW>), grid, dim3(NW * 64), 0, s, a);
    return NSV_OK;
  }
  return NSV_ERR_UNSUPPORTED;
}

// Head-dim slice width dc = D / dqc must be one the kernels are built for
// (32, or 64 when MT <= 2): the grid's dq index times DC must stay inside
// the head, so any other slicing is refused before launch.
template <int MT>
int launch_bf16(const VerifyArgs& a, int D, dim3 grid, hipStream_t s) {
  if (a.dqc <= 0 || D % a.dqc) return NSV_ERR_UNSUPPORTED;
  const int dc = D / a.dqc;
  if (dc == 32) {
    if (D == 128) launch_bf16_dc<MT, 128, 32>(a, grid, s);
    else launch_bf16_dc<MT, 64, 32>(a, grid, s);
    return NSV_OK;
  }
  if constexpr (MT <= 2) {
    if (dc == 64) {
      if (D == 128) launch_bf16_dc<MT, 128, 64>(a, grid, s);
      else launch_bf16_dc<MT, 64, 64>(a, grid, s);
      return NSV_OK;
    }
  }
  return NSV_ERR_UNSUPPORTED;
}

// fp32: at most two 16-row tiles per launch; more query rows per pair run
// as further launches over the next 32 rows (the single-launch form for 64
// rows, 256 VGPRs + 254 AGPRs of row state per lane, returned wrong rows on
// MI355X; two launches read the pair's K/V twice, which the 1e-5 path can
// afford).
template <int MT>
void launch_f32(const VerifyArgs& a, int D, dim3 grid, hipStream_t s) {
  if constexpr (MT <= 2) {
    if (D == 128)
      hipLaunchKernelGGL((verify_attn_f32_kernel<MT, 128>), grid, dim3(64), 0, s, a);
    else
      hipLaunchKernelGGL((verify_attn_f32_kernel<MT, 64>), grid, dim3(64), 0, s, a);
  } else {
    VerifyArgs b = a;
    b.m_base = 0;
    launch_f32<2>(b, D, grid, s);
    b.m_base = 32;
    launch_f32<MT - 2>(b, D, grid, s);
  }
}

// ---------------------------------------------------------------------------
// Load-only measurement kernels (the ceilings bench.py --ceiling reports).
// ---------------------------------------------------------------------------
// attn_load_floor_kernel reads exactly the K/V bytes of the key-split kernel,
// in its access pattern: workgroup = (pair, key split) with every split of a
// pair on one XCD, the block-table row staged in LDS first, then each of the
// 8 waves streams its interleaved 16-key tiles (K and V rows of one kv head,
// whole 256-byte rows, 4 + 4 loads of 16 bytes per lane) with one tile in
// flight.  Nothing is computed; the loaded words are folded into one value
// written only if it equals a constant no input produces in practice.
__global__ __launch_bounds__(512) void attn_load_floor_kernel(VerifyArgs a, uint32_t* sink) {
  const int wg = blockIdx.x;
  const int yy = wg >> 3;
  const int pair = (yy % a.P8) * 8 + (wg & 7);
  const int split = yy / a.P8;
  if (pair >= a.npairs) return;
  const int b = pair / a.Hkv, hk = pair - b * a.Hkv;
  __shared__ int pages[kMaxSplitPages];
  for (int j = threadIdx.x; j < a.max_blocks; j += 512) pages[j] = a.block_tables[(int64_t)b * a.max_blocks + j];
  const int ctx = context_len(a, b);
  __syncthreads();
  const int nsplit = num_splits(a, ctx);
  if (split >= nsplit) return;
  const int len = split_len(a, ctx);
  const int kb = split * len, ke = min(ctx, kb + len);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ntiles = (ke - kb + 15) / 16;
  const unsigned row_bytes = (unsigned)a.Hkv * 256;
  const int bs_mask = (1 << a.bs_log2) - 1;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int t = w; t < ntiles; t += 8) {
    const int n0 = kb + t * 16;
    const int pg = pages[n0 >> a.bs_log2];
    if (pg < 0) continue;
    const size_t base = ((size_t)pg << a.bs_log2) * row_bytes + (size_t)hk * 256 + (lane & 15) * 16;
    u32x4 kv[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int key = ((n0 & bs_mask) + j * 4 + (lane >> 4));
      kv[j] = load16_stream((const char*)a.k_cache + base + (size_t)key * row_bytes);
      kv[4 + j] = load16_stream((const char*)a.v_cache + base + (size_t)key * row_bytes);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= kv[j];
  }
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x9e3779b9u) sink[blockIdx.x] = x;
}

// Contiguous read of `bytes` in equal per-workgroup chunks, 4 loads of 16
// bytes per lane in flight: the streaming ceiling at a given size.
__global__ __launch_bounds__(512) void stream_read_kernel(const char* buf, size_t per, size_t bytes, uint32_t* sink) {
  const size_t beg = (size_t)blockIdx.x * per;
  const size_t end = beg + per < bytes ? beg + per : bytes;
  u32x4 acc = {0u, 0u, 0u, 0u};
  constexpr size_t step = 512 * 16;
  size_t off = beg + threadIdx.x * 16;
  for (; off + 3 * step + 16 <= end; off += 4 * step) {
    u32x4 t[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) t[u] = load16_stream(buf + off + u * step);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= t[u];
  }
  for (; off + 16 <= end; off += step) acc ^= load16_stream(buf + off);
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x9e3779b9u) sink[blockIdx.x] = x;
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (nsv_verify_attention_noalloc).
// ---------------------------------------------------------------------------
// A fixed device array holds what the caller's workspace holds otherwise:
// the arrival-counter area, then the split partials.  Every device the
// library runs on gets its own copy, at its own address, for the life of
// the process.  Device globals start zeroed and every call leaves the
// counters zero, the invariant the workspace contract already relies on.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __attribute__((aligned(256))) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

__global__ void clear_counters_kernel(unsigned* counters, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) counters[i] = 0u;
}

// The current device's copy of `scratch`, looked up once per device with
// that device current (the array's name in host code is a host-side handle,
// not a device address).  The first lookup on a device also enqueues a
// clear of the counter area on `stream` (a kernel, so that a caller
// capturing the stream records no memset node).  Returns a hipError_t.
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return NSV_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    hipLaunchKernelGGL(clear_counters_kernel, dim3((kMaxCounterPairs + 255) / 256), dim3(256), 0, stream,
                       (unsigned*)ptr, kMaxCounterPairs);
    const int rc = nsv_launch_status();
    if (rc != NSV_OK) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return NSV_OK;
}

// The kernels of one verify-attention launch (the head subset a.g0 ..
// a.g0 + a.G - 1 of every kv head): the key-split kernel, or the d-sliced /
// fp32 kernel and, with key splits, the merge kernel.
int launch_verify(const VerifyArgs& a, const Plan& p, int D, int dtype, hipStream_t s) {
  int rc = NSV_OK;
  const dim3 grid(8 * p.S * a.P8 * p.dqc);
  if (dtype == NSV_BF16 && p.ks) {
    const dim3 kgrid(8 * a.P8, p.S);  // (pair, split)
    switch (p.MT) {
      case 1: rc = launch_ks<1>(a, D, kgrid, s); break;
      case 2: rc = launch_ks<2>(a, D, kgrid, s); break;
      default: rc = launch_ks<3>(a, D, kgrid, s); break;
    }
    if (rc != NSV_OK) return rc;
  } else if (dtype == NSV_BF16) {
    const dim3 dgrid(8 * a.P8, p.dqc, p.S);  // (pair, head-dim slice, split)
    switch (p.MT) {
      case 1: rc = launch_bf16<1>(a, D, dgrid, s); break;
      case 2: rc = launch_bf16<2>(a, D, dgrid, s); break;
      case 3: rc = launch_bf16<3>(a, D, dgrid, s); break;
      default: rc = launch_bf16<4>(a, D, dgrid, s); break;
    }
    if (rc != NSV_OK) return rc;
  } else {
    switch (p.MT) {
      case 1: launch_f32<1>(a, D, grid, s); break;
      case 2: launch_f32<2>(a, D, grid, s); break;
      case 3: launch_f32<3>(a, D, grid, s); break;
      default: launch_f32<4>(a, D, grid, s); break;
    }
  }
  rc = nsv_launch_status();
  if (rc != NSV_OK || p.S <= 1 || (dtype == NSV_BF16 && (p.ks || a.dmerge))) return rc;  // merged in-kernel
  const dim3 mgrid(a.npairs, (p.Mv + 3) / 4);
  if (dtype == NSV_BF16) {
    if (D == 128) hipLaunchKernelGGL((verify_merge_kernel<bf16_t, 2>), mgrid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((verify_merge_kernel<bf16_t, 1>), mgrid, dim3(256), 0, s, a);
  } else {
    if (D == 128) hipLaunchKernelGGL((verify_merge_kernel<float, 2>), mgrid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((verify_merge_kernel<float, 1>), mgrid, dim3(256), 0, s, a);
  }
  return nsv_launch_status();
}


#if NSV_STAMP
unsigned long long* g_stamp_buf = nullptr;  // [calls][kStampMaxWgs][kStampSlots]
int g_stamp_calls = 0;
unsigned g_stamp_next = 0;
#endif

}  // namespace

extern "C" {

int nsv_version(void) { return 100; }

int nsv_stamp_configure(void* buf, int calls) {
#if NSV_STAMP
  if (calls < 0 || (calls > 0 && !buf)) return NSV_ERR_ARG;
  g_stamp_buf = calls > 0 ? (unsigned long long*)buf : nullptr;
  g_stamp_calls = calls;
  g_stamp_next = 0;
  return NSV_OK;
#else
  (void)buf;
  (void)calls;
  return NSV_ERR_UNSUPPORTED;
#endif
}

const char* nsv_error_string(int code) {
  switch (code) {
    case NSV_OK: return "ok";
    case NSV_ERR_ARG: return "invalid argument";
    case NSV_ERR_UNSUPPORTED: return "unsupported shape";
    case NSV_ERR_WORKSPACE: return "workspace missing or too small";
    case NSV_ERR_SCRATCH: return "shape needs more scratch than the allocation-free entry point holds";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}

size_t nsv_verify_attention_workspace_size(int B, int H, int Hkv, int D, int block_size, int max_blocks,
                                           int max_q_len, int dtype, int kv_split_tokens) {
  Plan p;
  if (make_plan(B, H, Hkv, D, block_size, max_blocks, max_q_len, dtype, kv_split_tokens, device_cus(), &p) != NSV_OK)
    return 0;
  return workspace_bytes_for(B, Hkv, D, p);
}

int nsv_verify_attention_plan(int B, int H, int Hkv, int D, int block_size, int max_blocks, int max_q_len, int dtype,
                              int kv_split_tokens, int cus, int* kernel, int* splits) {
  Plan p;
  const int rc = make_plan(B, H, Hkv, D, block_size, max_blocks, max_q_len, dtype, kv_split_tokens,
                           cus > 0 ? cus : device_cus(), &p);
  if (rc != NSV_OK) return rc;
  if (kernel) *kernel = dtype == NSV_F32 ? NSV_ATTN_F32 : (p.ks ? NSV_ATTN_KEY_SPLIT : NSV_ATTN_DSLICED);
  if (splits) *splits = p.S;
  return NSV_OK;
}

int nsv_verify_attention(void* out, const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* block_tables, const int64_t* context_lens, const int32_t* cu_seqlens_q,
                         const int64_t* positions, float scale, int B, int T, int H, int Hkv, int D, int block_size,
                         int max_blocks, int max_q_len, int dtype, int kv_split_tokens, void* workspace,
                         size_t workspace_bytes, void* stream) {
  Plan p;
  int rc = make_plan(B, H, Hkv, D, block_size, max_blocks, max_q_len, dtype, kv_split_tokens, device_cus(), &p);
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
  char* ws = (char*)workspace;
  a.counters = need ? (unsigned*)ws : nullptr;
  a.part_ml = need ? (float*)(ws + counter_bytes(B, Hkv)) : nullptr;
  a.part_o = need ? (float*)(ws + counter_bytes(B, Hkv) + ml_bytes(B, Hkv, p)) : nullptr;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.H = H;
  a.Hkv = Hkv;
  a.G = p.G;
  a.Gs = p.Gs;
  a.g0 = 0;
  a.bs_log2 = ilog2_exact(block_size);
  a.max_blocks = max_blocks;
  a.QL = p.QL;
  a.Mv = p.Mv;
  a.S = p.S;
  a.split_tokens = p.split;
  a.npairs = B * Hkv;
  a.P8 = (B * Hkv + 7) / 8;
  a.dqc = p.dqc;
  a.ks_splits = p.ks_splits;
  a.m_base = 0;
  // the d-sliced kernel merges its key splits in-kernel while every pair has
  // an arrival counter of its own, else in a second launch
  a.dmerge = dtype == NSV_BF16 && !p.ks && p.S > 1 && (int64_t)B * Hkv * p.dqc <= kMaxCounterPairs;

  hipStream_t s = (hipStream_t)stream;
  // one launch (and merge) per subset of each kv head's query heads; they
  // share the workspace in stream order
  for (a.g0 = 0; a.g0 < p.Gs; a.g0 += p.G) {
#if NSV_STAMP
    a.stamps = nullptr;
    if (g_stamp_buf && 8 * p.S * a.P8 * p.dqc <= kStampMaxWgs)
      a.stamps = g_stamp_buf + (size_t)(g_stamp_next++ % (unsigned)g_stamp_calls) * kStampMaxWgs * kStampSlots;
#endif
    rc = launch_verify(a, p, D, dtype, s);
    if (rc != NSV_OK) return rc;
  }
  return NSV_OK;
}

int nsv_verify_attention_load_floor(const void* k_cache, const void* v_cache, const int32_t* block_tables,
                                    const int64_t* context_lens, int B, int Hkv, int D, int block_size,
                                    int max_blocks, int splits, void* sink, void* stream) {
  if (B < 0 || Hkv <= 0 || max_blocks <= 0 || splits <= 0 || splits > 64) return NSV_ERR_ARG;
  if (D != 128 || ilog2_exact(block_size) < 4 || max_blocks > kMaxSplitPages) return NSV_ERR_UNSUPPORTED;
  if (B == 0) return NSV_OK;
  if (!k_cache || !v_cache || !block_tables || !context_lens || !sink) return NSV_ERR_ARG;
  VerifyArgs a{};
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.block_tables = block_tables;
  a.context_lens = context_lens;
  a.Hkv = Hkv;
  a.bs_log2 = ilog2_exact(block_size);
  a.max_blocks = max_blocks;
  a.npairs = B * Hkv;
  a.P8 = (B * Hkv + 7) / 8;
  a.split_tokens = 0;
  a.ks_splits = splits;
  hipLaunchKernelGGL(attn_load_floor_kernel, dim3(8 * splits * a.P8), dim3(512), 0, (hipStream_t)stream, a,
                     (uint32_t*)sink);
  return nsv_launch_status();
}

int nsv_stream_read(const void* buf, size_t bytes, int workgroups, void* sink, void* stream) {
  if (!buf || !sink || workgroups <= 0 || (bytes % 16)) return NSV_ERR_ARG;
  if (bytes == 0) return NSV_OK;
  const size_t per = ((bytes + workgroups - 1) / workgroups + 15) & ~(size_t)15;
  hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(512), 0, (hipStream_t)stream, (const char*)buf, per,
                     bytes, (uint32_t*)sink);
  return nsv_launch_status();
}

size_t nsv_verify_attention_noalloc_max_scratch(void) { return kNoAllocScratchBytes; }

int nsv_verify_attention_noalloc(void* out, const void* q, const void* k_cache, const void* v_cache,
                                 const int32_t* block_tables, const int64_t* context_lens,
                                 const int32_t* cu_seqlens_q, const int64_t* positions, float scale, int B, int T,
                                 int H, int Hkv, int D, int block_size, int max_blocks, int max_q_len, int dtype,
                                 int kv_split_tokens, void* stream) {
  Plan p;
  int rc = make_plan(B, H, Hkv, D, block_size, max_blocks, max_q_len, dtype, kv_split_tokens, device_cus(), &p);
  if (rc != NSV_OK) return rc;
  if (workspace_bytes_for(B, Hkv, D, p) > kNoAllocScratchBytes) return NSV_ERR_SCRATCH;
  void* ws = nullptr;
  rc = scratch_for_current_device((hipStream_t)stream, &ws);
  if (rc != NSV_OK) return rc;
  return nsv_verify_attention(out, q, k_cache, v_cache, block_tables, context_lens, cu_seqlens_q, positions, scale,
                              B, T, H, Hkv, D, block_size, max_blocks, max_q_len, dtype, kv_split_tokens, ws,
                              kNoAllocScratchBytes, stream);
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
