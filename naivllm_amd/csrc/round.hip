// Device-side bookkeeping of the verification round for gfx950: builds the
// verify forward's per-row metadata from the device-resident token history
// and drafts, and commits the accepted tokens back into the history.  With
// these two kernels (plus the drafter, the forward and the acceptance
// kernels) a whole round runs without the host and is captured in one
// hipGraph.
//
// prepare: src/myvllm/engine/model_runner.py:734-774 (_run_spec_verify_graph
//   row building: inputs [last_confirmed, d_1..d_K] at positions n-1..n+K-1,
//   slot = table[pos / bs] * bs + pos % bs, context length n + K, pad rows
//   (id 0, position -1, slot -1) up to K+1 rows per sequence).
// commit: src/myvllm/spec_engine/spec_llm_engine.py:249-291 (_commit: cap by
//   max_tokens, stop at eos unless ignore_eos, stop at max_model_length,
//   then the finish test).
// prepare_draft: the per-step rows of a model drafter's K decode steps
//   (engine/model_runner.py:784-823, run_draft_steps_gpu), all steps in one
//   launch.

#include "common.h"

namespace {

struct PrepareArgs {
  const int32_t* history;    // [B, hstride]
  int64_t hstride;
  const int32_t* hist_len;   // [B]
  const int32_t* drafts;     // [B, K]
  const int32_t* num_drafts; // [B]
  const int32_t* block_tables;  // [B, max_blocks]
  const int32_t* active;     // [B] 0: finished or empty slot
  int B, K, max_blocks, block_size;
  int64_t* input_ids;        // [B*(K+1)]
  int64_t* positions;        // [B*(K+1)]
  int64_t* slot_mapping;     // [B*(K+1)]
  int64_t* context_lens;     // [B]
};

__global__ __launch_bounds__(64) void prepare_verify_kernel(PrepareArgs a) {
  const int b = blockIdx.x, j = threadIdx.x;
  const int R = a.K + 1;
  if (j >= R) return;
  const int64_t row = (int64_t)b * R + j;
  const int n = a.hist_len[b];
  const int k = min(max(a.num_drafts[b], 0), a.K);
  const bool live = a.active[b] && n > 0 && j <= k;
  if (j == 0) a.context_lens[b] = (a.active[b] && n > 0) ? n + k : 0;
  if (!live) {
    a.input_ids[row] = 0;
    a.positions[row] = -1;
    a.slot_mapping[row] = -1;
    return;
  }
  const int pos = n - 1 + j;
  const int tok = j == 0 ? a.history[(int64_t)b * a.hstride + n - 1] : a.drafts[(int64_t)b * a.K + j - 1];
  const int page = a.block_tables[(int64_t)b * a.max_blocks + pos / a.block_size];
  a.input_ids[row] = tok;
  a.positions[row] = pos;
  a.slot_mapping[row] = page < 0 ? -1 : (int64_t)page * a.block_size + pos % a.block_size;
}

struct DraftPrepArgs {
  const int32_t* history;    // [B, hstride]
  int64_t hstride;
  const int32_t* hist_len;   // [B]
  const int32_t* block_tables;  // [B, max_blocks] (the draft model's pages)
  const int32_t* active;     // [B]
  int B, K, max_blocks, block_size;
  int64_t* ids0;             // [2B] step 0: the last two confirmed tokens of each sequence
  int64_t* pos0;             // [2B]
  int64_t* slot0;            // [2B]
  int64_t* pos;              // [K, B] position of step i's row (i >= 1)
  int64_t* slot;             // [K, B]
  int64_t* ctx;              // [K, B] context length of step i
};

// Step i of sequence b (n confirmed tokens) feeds the token at position
// n-1+i and attends keys 0..n-1+i.  Step 0 also re-feeds the token at n-2:
// after a round whose drafts were all accepted, that token (the last draft)
// was never fed to the drafter, and this row writes its draft-cache entry.
__global__ __launch_bounds__(64) void prepare_draft_kernel(DraftPrepArgs a) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  const int n = a.hist_len[b];
  const bool live = a.active[b] && n > 0;
  auto slot_of = [&](int pos) -> int64_t {
    const int page = a.block_tables[(int64_t)b * a.max_blocks + pos / a.block_size];
    return page < 0 ? -1 : (int64_t)page * a.block_size + pos % a.block_size;
  };
  for (int j = 0; j < 2; ++j) {
    const int pos = n - 2 + j;
    const bool ok = live && pos >= 0;
    a.ids0[2 * b + j] = ok ? a.history[(int64_t)b * a.hstride + pos] : 0;
    a.pos0[2 * b + j] = ok ? pos : -1;
    a.slot0[2 * b + j] = ok ? slot_of(pos) : -1;
  }
  for (int i = 0; i < a.K; ++i) {
    const int pos = n - 1 + i;
    const int64_t r = (int64_t)i * a.B + b;
    a.pos[r] = live ? pos : -1;
    a.slot[r] = live ? slot_of(pos) : -1;
    a.ctx[r] = live ? pos + 1 : 0;
  }
}

struct CommitArgs {
  const int32_t* tokens;     // [B, K+1] accepted tokens
  const int32_t* num_tokens; // [B]
  const int32_t* num_drafts; // [B]
  int32_t* history;          // [B, hstride]
  int64_t hstride;
  int32_t* hist_len;         // [B]
  const int32_t* prompt_len; // [B]
  const int32_t* max_tokens; // [B]
  const int32_t* max_len;    // [B] max_model_length, <= 0: none
  const int32_t* ignore_eos; // [B]
  int32_t* active;           // [B] cleared when the sequence finishes
  int32_t* committed;        // [B] tokens appended this round
  int B, K, eos;
};

__global__ __launch_bounds__(64) void commit_kernel(CommitArgs a) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  a.committed[b] = 0;
  if (!a.active[b]) return;
  const int n = a.hist_len[b];
  const int completed = n - a.prompt_len[b];
  const int allowed = max(0, a.max_tokens[b] - completed);
  const int m = min(min(a.num_tokens[b], a.K + 1), allowed);
  int c = 0;
  int last = -1;
  for (int i = 0; i < m; ++i) {
    const int t = a.tokens[(int64_t)b * (a.K + 1) + i];
    if (n + c >= a.hstride) break;  // history buffer full
    a.history[(int64_t)b * a.hstride + n + c] = t;
    ++c;
    last = t;
    const bool eos = !a.ignore_eos[b] && t == a.eos;
    const bool length = a.max_len[b] > 0 && n + c >= a.max_len[b];
    if (eos || length) break;
  }
  a.hist_len[b] = n + c;
  a.committed[b] = c;
  const bool stop_eos = c > 0 && !a.ignore_eos[b] && last == a.eos;
  const bool stop_tokens = n + c - a.prompt_len[b] >= a.max_tokens[b];
  const bool stop_len = a.max_len[b] > 0 && n + c >= a.max_len[b];
  const bool full = n + c + a.K + 1 > a.hstride;  // no room for another round
  if (stop_eos || stop_tokens || stop_len || full) a.active[b] = 0;
}

}  // namespace

extern "C" {

int nsv_prepare_verify(const int32_t* history, int64_t hist_stride, const int32_t* hist_len, const int32_t* drafts,
                       const int32_t* num_drafts, const int32_t* block_tables, int max_blocks, int block_size,
                       const int32_t* active, int B, int K, int64_t* input_ids, int64_t* positions,
                       int64_t* slot_mapping, int64_t* context_lens, void* stream) {
  if (B < 0 || K < 0 || K + 1 > 64 || max_blocks <= 0 || block_size <= 0) return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!history || !hist_len || (!drafts && K > 0) || !num_drafts || !block_tables || !active || !input_ids ||
      !positions || !slot_mapping || !context_lens)
    return NSV_ERR_ARG;
  PrepareArgs a{history, hist_stride, hist_len, drafts, num_drafts, block_tables, active, B, K, max_blocks,
                block_size, input_ids, positions, slot_mapping, context_lens};
  hipLaunchKernelGGL(prepare_verify_kernel, dim3(B), dim3(64), 0, (hipStream_t)stream, a);
  return nsv_launch_status();
}

int nsv_prepare_draft(const int32_t* history, int64_t hist_stride, const int32_t* hist_len,
                      const int32_t* block_tables, int max_blocks, int block_size, const int32_t* active, int B,
                      int K, int64_t* ids0, int64_t* pos0, int64_t* slot0, int64_t* positions,
                      int64_t* slot_mapping, int64_t* context_lens, void* stream) {
  if (B < 0 || K < 1 || max_blocks <= 0 || block_size <= 0 || hist_stride <= 0) return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!history || !hist_len || !block_tables || !active || !ids0 || !pos0 || !slot0 || !positions ||
      !slot_mapping || !context_lens)
    return NSV_ERR_ARG;
  DraftPrepArgs a{history, hist_stride, hist_len, block_tables, active, B, K, max_blocks, block_size,
                  ids0, pos0, slot0, positions, slot_mapping, context_lens};
  hipLaunchKernelGGL(prepare_draft_kernel, dim3((B + 63) / 64), dim3(64), 0, (hipStream_t)stream, a);
  return nsv_launch_status();
}

int nsv_commit(const int32_t* tokens, const int32_t* num_tokens, const int32_t* num_drafts, int32_t* history,
               int64_t hist_stride, int32_t* hist_len, const int32_t* prompt_len, const int32_t* max_tokens,
               const int32_t* max_len, const int32_t* ignore_eos, int eos, int32_t* active, int32_t* committed,
               int B, int K, void* stream) {
  if (B < 0 || K < 0 || hist_stride <= 0) return NSV_ERR_ARG;
  if (B == 0) return NSV_OK;
  if (!tokens || !num_tokens || !history || !hist_len || !prompt_len || !max_tokens || !max_len || !ignore_eos ||
      !active || !committed)
    return NSV_ERR_ARG;
  CommitArgs a{tokens, num_tokens, num_drafts, history, hist_stride, hist_len, prompt_len, max_tokens, max_len,
               ignore_eos, active, committed, B, K, eos};
  hipLaunchKernelGGL(commit_kernel, dim3((B + 63) / 64), dim3(64), 0, (hipStream_t)stream, a);
  return nsv_launch_status();
}

}  // extern "C"
