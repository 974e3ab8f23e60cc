// GPU n-gram (prompt-lookup) drafter for gfx950.
//
// Behaviour follows NgramDrafter._lookup (src/myvllm/spec_engine/
// drafters.py:63-83), which searches the big-endian uint32 byte encoding of
// the token history with bytes.rfind.  The kernel reproduces that byte-level
// search exactly, including hits at byte offsets inside a token (which move
// the search end left of them and make the reference skip aligned matches
// that overlap them), without building the byte string: the 32-bit word at
// byte offset 4i + r is (h[i] << 8r) | (h[i+1] >> (32 - 8r)).
//
// One workgroup per sequence; the history is staged in LDS when it fits.
// For n = min(max_n, L-1) down to min_n, the workgroup scans byte offsets
// from the highest allowed one downwards, 256 offsets per step, each thread
// testing one offset; the highest matching offset of a step ends the scan.

#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kHistLds = 12288;  // tokens of history staged in LDS (48 KB)
constexpr int kMaxN = 64;        // longest n-gram
constexpr int kMaxK = 64;        // longest continuation

struct NgramArgs {
  const int32_t* history;  // [B, stride]
  const int32_t* hist_len; // [B]
  int64_t stride;
  int B, min_n, max_n, K;
  int32_t* out_drafts;     // [B, K]
  int32_t* out_len;        // [B]
};

__global__ __launch_bounds__(kThreads) void ngram_draft_kernel(NgramArgs a) {
  __shared__ uint32_t hs[kHistLds];
  __shared__ uint32_t needle[kMaxN];
  __shared__ int red[kThreads / 64];
  const int b = blockIdx.x, tid = threadIdx.x;
  const uint32_t* hg = (const uint32_t*)a.history + (int64_t)b * a.stride;
  const int L = max(0, (int)min((int64_t)a.hist_len[b], a.stride));
  const bool in_lds = L <= kHistLds;
  if (in_lds)
    for (int i = tid; i < L; i += kThreads) hs[i] = hg[i];
  __syncthreads();
  auto tok = [&](int i) -> uint32_t { return in_lds ? hs[i] : hg[i]; };
  // big-endian 32-bit word at byte offset o (o + 4 <= 4L)
  auto word = [&](int o) -> uint32_t {
    const int i = o >> 2, r = o & 3;
    const uint32_t hi = tok(i);
    return r == 0 ? hi : (hi << (8 * r)) | (tok(i + 1) >> (32 - 8 * r));
  };

  const int nmax = min(min(a.max_n, L - 1), kMaxN);
  for (int n = nmax; n >= a.min_n && n >= 1; --n) {
    for (int m = tid; m < n; m += kThreads) needle[m] = tok(L - n + m);
    __syncthreads();
    int end = 4 * (L - 1);  // matches must end at or before this byte
    int found = -1;
    while (true) {
      // highest offset o <= end - 4n whose 4n bytes equal the needle
      int hit = -1;
      for (int top = end - 4 * n; top >= 0 && hit < 0; top -= kThreads) {
        const int o = top - tid;
        bool ok = o >= 0;
        for (int m = 0; ok && m < n; ++m) ok = word(o + 4 * m) == needle[m];
        // the highest matching offset of this step = the lowest matching tid
        const uint64_t bal = __ballot(ok);
        const int w = tid >> 6, lane = tid & 63;
        if (lane == 0) red[w] = bal ? (int)(__builtin_ctzll(bal)) + w * 64 : 0x7fffffff;
        __syncthreads();
        int best = 0x7fffffff;
        for (int i = 0; i < kThreads / 64; ++i) best = min(best, red[i]);
        __syncthreads();
        if (best != 0x7fffffff) hit = top - best;
      }
      if (hit < 0 || (hit & 3) == 0) {
        found = hit;
        break;
      }
      end = hit;  // a hit inside a token: search again left of it
    }
    if (found >= 0) {
      const int start = found / 4 + n;
      const int cnt = min(a.K, L - start);  // >= 1: the match ends before the last token
      for (int j = tid; j < cnt; j += kThreads) a.out_drafts[(int64_t)b * a.K + j] = (int32_t)tok(start + j);
      if (tid == 0) a.out_len[b] = cnt;
      return;
    }
    __syncthreads();  // before the next n rewrites the needle
  }
  if (tid == 0) a.out_len[b] = 0;
}

}  // namespace

extern "C" {

int nsv_ngram_draft(const int32_t* history, const int32_t* hist_len, int64_t hist_stride, int B, int min_n,
                    int max_n, int K, int32_t* out_drafts, int32_t* out_len, void* stream) {
  if (B < 0 || hist_stride < 0 || min_n < 1 || max_n < min_n || max_n > kMaxN || K < 1 || K > kMaxK)
    return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!history || !hist_len || !out_drafts || !out_len) return NSV_ERR_ARG;
  if (hist_stride > ((int64_t)1 << 29)) return NSV_ERR_UNSUPPORTED;  // byte offsets stay in int range
  NgramArgs a;
  a.history = history;
  a.hist_len = hist_len;
  a.stride = hist_stride;
  a.B = B;
  a.min_n = min_n;
  a.max_n = max_n;
  a.K = K;
  a.out_drafts = out_drafts;
  a.out_len = out_len;
  hipLaunchKernelGGL(ngram_draft_kernel, dim3(B), dim3(kThreads), 0, (hipStream_t)stream, a);
  return nsv_launch_status();
}

}  // extern "C"
