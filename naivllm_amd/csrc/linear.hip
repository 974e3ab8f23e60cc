// Few-row linear layers of the Qwen3 verify forward for gfx950 (bf16 in,
// fp32 accumulation, one bf16 rounding per output).
//
// The verify forward multiplies B*(K+1) activation rows (72 at batch 8) by weight
// matrices of 2-300 MB, so streaming the weights, not arithmetic, bounds
// every projection.  A workgroup owns 16 output columns (16 weight rows):
// its 8 waves take 128-element chunks of the reduction dimension in turn,
// load their slice of the 16
// rows as whole-row 16-byte loads (16 lanes cover 256 contiguous bytes of
// one row), reshape it through a per-wave LDS tile into the MFMA operand
// layout and multiply it with every activation row
// (v_mfma_f32_16x16x32_bf16, rows padded to 16; more than 80 rows take
// further workgroup rows of the grid); the waves' partial
// products are summed through LDS.  The next chunk's loads are issued
// before the current chunk is multiplied.
//
// Fused stages (each removes a kernel launch and an activation round trip):
//   * prologue RMSNorm (norm_w != NULL): the activation row is
//     rmsnorm(r) * norm_w with r the bf16 residual stream; sum(r^2) per row
//     arrives as per-tile partial sums from the producing linear and is
//     added in a fixed order;
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
constexpr int kKC = 128;           // reduction elements per wave chunk
constexpr int kWStr = kKC + 8;     // staged weight row stride (bf16): 272 bytes, distinct banks per row
constexpr int kMaxRows = 80;       // activation rows (5 MFMA row tiles)

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
};

__device__ __forceinline__ bf16x8 to_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ float bfv(uint32_t word, int hi) { return __uint_as_float(hi ? (word & 0xffff0000u) : (word << 16)); }

template <int MT, bool NORM, int EPI>  // EPI 0: plain, 1: SwiGLU, 2: residual
__global__ __launch_bounds__(kLinThreads) void linear_kernel(LinearArgs a) {
  constexpr int MP = MT * 16;
  constexpr int WST = kLinWaves * kBN * kWStr * 2;       // staged weight chunks, bytes
  constexpr int RED = kLinWaves * MP * (kBN + 1) * 4;    // cross-wave partial products, bytes
  constexpr int SMEM = WST > RED ? WST : RED;
  __shared__ __attribute__((aligned(16))) unsigned char smem[SMEM];
  __shared__ float inv_s[MP];
  __shared__ float ss_s[kLinThreads];

  const int tile = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, c = lane & 15;
  const int K = a.K;
  // rows of this workgroup: chunk blockIdx.y of kMaxRows rows
  const int row0 = blockIdx.y * kMaxRows;
  const int M = min(a.M - row0, kMaxRows);

  // weight row of tile column cc
  const int half = a.N >> 1;
  auto wrow = [&](int cc) -> int64_t {
    if constexpr (EPI == 1) return cc < 8 ? tile * 8 + cc : half + tile * 8 + (cc - 8);
    else return (int64_t)tile * kBN + cc;
  };
  // the reduction in chunks of kKC elements, dealt to the waves round-robin
  // (chunk w + 8i is wave w's i-th); a last partial chunk reads zeros past K
  const int nck = (K + kKC - 1) / kKC;
  const int nchunk = w < nck ? (nck - w + kLinWaves - 1) / kLinWaves : 0;
  const uint16_t* wrows[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) wrows[j] = a.w + wrow(4 * j + g4) * K + c * 8;

  struct Chunk {
    u32x4 wv[4];          // weight rows 4j + g4, elements 8c .. 8c+7 of the chunk
    u32x4 xv[MT][4];      // activation row 16mt + c, elements 32s + 8g4 .. +7
    u32x4 nv[4];          // RMSNorm weight, elements 32s + 8g4 .. +7
    int k0;
  };
  // PX: the activation slice of the next chunk is prefetched with its
  // weights (all but the widest normalising instances, whose registers
  // would not hold two chunks; those load it when the chunk is multiplied)
  constexpr bool PX = !(NORM && MT >= 4);
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  auto issue_x = [&](Chunk& ch, int k0) {
    const bool whole = k0 + kKC <= K;  // uniform
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + c;
      const uint16_t* xr = a.x + (int64_t)(row0 + (m < M ? m : M - 1)) * K + k0 + 8 * g4;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        ch.xv[mt][s] = (whole || k0 + 32 * s + 8 * g4 < K) ? *reinterpret_cast<const u32x4*>(xr + 32 * s) : zero4;
    }
    if constexpr (NORM) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        ch.nv[s] = (whole || k0 + 32 * s + 8 * g4 < K) ? *reinterpret_cast<const u32x4*>(a.norm_w + k0 + 32 * s + 8 * g4)
                                                        : zero4;
    }
  };
  auto issue = [&](Chunk& ch, int k0) {
    const bool whole = k0 + kKC <= K;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      ch.wv[j] = (whole || k0 + c * 8 < K) ? *reinterpret_cast<const u32x4*>(wrows[j] + k0) : zero4;
    ch.k0 = k0;
    if constexpr (PX) issue_x(ch, k0);
  };

  uint16_t* wst = reinterpret_cast<uint16_t*>(smem) + w * kBN * kWStr;
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  float rowinv[MT];  // 1 / rms of each row of the lane's row tiles (RMSNorm prologue)
  auto compute = [&](Chunk& ch) {
    if constexpr (!PX) issue_x(ch, ch.k0);
    // stage the 16 weight rows of the chunk (this wave's LDS rows)
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(wst + (4 * j + g4) * kWStr + c * 8) = ch.wv[j];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const u32x4 bw = *reinterpret_cast<const u32x4*>(wst + c * kWStr + 32 * s + 8 * g4);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        u32x4 av = ch.xv[mt][s];
        if (mt * 16 + c >= M) av = u32x4{0u, 0u, 0u, 0u};
        if constexpr (NORM) {
          // h = bf16(r * inv * norm_w), the RMSNorm output the projection consumes
          uint32_t o[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float h0 = bfv(av[q], 0) * rowinv[mt] * bfv(ch.nv[s][q], 0);
            const float h1 = bfv(av[q], 1) * rowinv[mt] * bfv(ch.nv[s][q], 1);
            o[q] = (uint32_t)f32_to_bf16_bits(h0) | ((uint32_t)f32_to_bf16_bits(h1) << 16);
          }
          av = u32x4{o[0], o[1], o[2], o[3]};
        }
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(to_bf16x8(av), to_bf16x8(bw), acc[mt], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- two-stage pipeline over this wave's chunks
  Chunk A, B;
  auto k_of = [&](int i) { return (w + i * kLinWaves) * kKC; };
  if (nchunk > 0) issue(A, k_of(0));  // the first weights stream in during the prologue below

  // ---- RMSNorm prologue: 1 / rms per row from the producer's partial sums,
  // added in a fixed order (thread part p sums slots p, p + P, ...; row m
  // then sums the P part sums in order)
  if constexpr (NORM) {
    constexpr int P = kLinThreads / MP;
    const int m = tid % MP, p = tid / MP;
    float s = 0.f;
    if (p < P && m < M)
      for (int j = p; j < a.nss_in; j += P) s += a.ss_in[(int64_t)j * a.M + row0 + m];
    ss_s[tid] = s;
    __syncthreads();
    if (tid < MP) {
      float t = 0.f;
      for (int q = 0; q < P; ++q) t += ss_s[q * MP + tid];
      inv_s[tid] = rsqrtf(t / (float)K + a.eps);
    }
    __syncthreads();
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) rowinv[mt] = NORM ? inv_s[mt * 16 + c] : 1.f;

  for (int i = 0; i < nchunk; i += 2) {
    if (i + 1 < nchunk) issue(B, k_of(i + 1));
    compute(A);
    if (i + 1 < nchunk) {
      if (i + 2 < nchunk) issue(A, k_of(i + 2));
      compute(B);
    }
  }

  // ---- sum the waves' partial products: lane (g4, c) holds C[16mt + 4g4 + i][c]
  __syncthreads();  // every wave is done with its staged weights (red aliases them)
  float* red = reinterpret_cast<float*>(smem);  // [kLinWaves][MP][kBN + 1]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(w * MP + mt * 16 + g4 * 4 + i) * (kBN + 1) + c] = acc[mt][i];
  __syncthreads();
  auto colsum = [&](int m, int col) {
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < kLinWaves; ++ww) v += red[(ww * MP + m) * (kBN + 1) + col];
    return v;
  };
  if constexpr (EPI == 1) {
    // item = (row, 4 gate columns): silu(gate) * up for 4 outputs
    if (tid < MP * 2) {
      const int m = tid >> 1, q = tid & 1;
      if (m < M) {
        uint32_t o[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float r2[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int col = 4 * q + 2 * j + e;
            const float g = bf16_bits_to_f32(f32_to_bf16_bits(colsum(m, col)));
            const float u = bf16_bits_to_f32(f32_to_bf16_bits(colsum(m, 8 + col)));
            r2[e] = g / (1.f + __expf(-g)) * u;
          }
          o[j] = (uint32_t)f32_to_bf16_bits(r2[0]) | ((uint32_t)f32_to_bf16_bits(r2[1]) << 16);
        }
        *reinterpret_cast<uint2*>(a.y + (int64_t)(row0 + m) * half + tile * 8 + 4 * q) = make_uint2(o[0], o[1]);
      }
    }
  } else {
    // item = (row, 4 columns)
    const int m = tid >> 2, q = tid & 3;
    float ss = 0.f;
    if (tid < MP * 4 && m < M) {
      const int64_t off = (int64_t)(row0 + m) * a.N + (int64_t)tile * kBN + 4 * q;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = bf16_bits_to_f32(f32_to_bf16_bits(colsum(m, 4 * q + e)));
      uint16_t* dst = EPI == 2 ? a.resid : a.y;
      if constexpr (EPI == 2) {
        const uint2 rv = *reinterpret_cast<const uint2*>(a.resid + off);
        const uint32_t rw[2] = {rv.x, rv.y};
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
      // the 4 threads of a row are lanes 4m' .. 4m'+3 of one wave: fixed-order butterfly
      ss += __shfl_xor(ss, 1, NSV_WAVE);
      ss += __shfl_xor(ss, 2, NSV_WAVE);
      if (tid < MP * 4 && m < M && q == 0) a.ss_out[(int64_t)tile * a.M + row0 + m] = ss;
    }
  }
}

template <int MT>
int launch_linear(const LinearArgs& a, bool norm, int epi, dim3 grid, hipStream_t s) {
#define NSV_LIN(NORM, EPI) hipLaunchKernelGGL((linear_kernel<MT, NORM, EPI>), grid, dim3(kLinThreads), 0, s, a)
  if (norm) {
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

}  // namespace

extern "C" {

int nsv_linear(const void* x, const void* norm_w, const float* ss_in, int nss_in, float eps, const void* weight,
               void* y, void* resid, float* ss_out, int M, int N, int K, int epilogue, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || epilogue < 0 || epilogue > 2) return NSV_ERR_ARG;
  if (M == 0) return NSV_OK;
  if (N % kBN || K % 8 || M > 65535 * kMaxRows) return NSV_ERR_UNSUPPORTED;
  if (!x || !weight) return NSV_ERR_ARG;
  if (norm_w && (!ss_in || nss_in <= 0)) return NSV_ERR_ARG;
  if (epilogue == 2 ? (!resid || !ss_out) : !y) return NSV_ERR_ARG;
  LinearArgs a{(const uint16_t*)x, (const uint16_t*)norm_w, ss_in, nss_in, eps, (const uint16_t*)weight,
               (uint16_t*)y, (uint16_t*)resid, ss_out, M, N, K};
  const dim3 grid(N / kBN, (M + kMaxRows - 1) / kMaxRows);
  hipStream_t s = (hipStream_t)stream;
  const bool norm = norm_w != nullptr;
  switch ((min(M, kMaxRows) + 15) / 16) {
    case 1: return launch_linear<1>(a, norm, epilogue, grid, s);
    case 2: return launch_linear<2>(a, norm, epilogue, grid, s);
    case 3: return launch_linear<3>(a, norm, epilogue, grid, s);
    case 4: return launch_linear<4>(a, norm, epilogue, grid, s);
    default: return launch_linear<5>(a, norm, epilogue, grid, s);
  }
}

}  // extern "C"
