/*
 * naivspec.h — C ABI of libnaivspec.so, the MI355X (gfx950) kernels of the
 * speculative-decoding verification round.
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are caller-owned device pointers, row-major and
 *     contiguous unless a stride argument says otherwise.
 *   - `stream` is a hipStream_t passed as void* (torch's
 *     torch.cuda.current_stream().cuda_stream); work is enqueued there and
 *     never synchronised, so every call can be captured into a hipGraph.
 *   - No entry point allocates device memory.  Scratch comes in through an
 *     explicit `workspace` pointer sized by the matching *_workspace_size().
 *   - Return value: 0 on success, a negative NSV_ERR_* code for a rejected
 *     argument (nothing was launched), or a positive hipError_t when the
 *     launch itself failed.
 *   - dtype codes: NSV_F32 = 0, NSV_BF16 = 1.
 *
 * Each declaration cites the reference interface (Hongli-xd/Naivllm,
 * src/myvllm/...) whose behaviour it reproduces.
 */
#ifndef NAIVSPEC_H
#define NAIVSPEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSV_F32 0
#define NSV_BF16 1

#define NSV_OK 0
#define NSV_ERR_ARG (-1)         /* null pointer, negative size, bad dtype  */
#define NSV_ERR_UNSUPPORTED (-2) /* shape outside what the kernels handle   */
#define NSV_ERR_WORKSPACE (-3)   /* workspace pointer null or too small     */
#define NSV_ERR_SCRATCH (-4)     /* shape beyond the allocation-free entry  */
                                 /* point's fixed scratch                    */

/* Library version (major*10000 + minor*100 + patch). */
int nsv_version(void);

/* Human-readable text for a return code of any nsv_* function. */
const char* nsv_error_string(int code);

/*
 * Paged multi-token verify attention.
 * Replaces layers/attention.py:615-668 (paged_attention_verify) and its
 * Triton kernel :522-612.  For query row r of sequence b (rows
 * cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1) and head h:
 *     out[r,h,:] = softmax_j(scale * q[r,h,:] . k_j) V_j
 * over keys j <= positions[r], j < context_lens[b], whose page
 * block_tables[b, j / block_size] is >= 0; kv head = h / (H / Hkv).
 * Rows with positions[r] < 0 (inert padding) are written as zeros.
 *   q, out        [T, H, D]              dtype
 *   k_cache/v_cache  [num_blocks, block_size, Hkv, D] (one layer), dtype
 *   block_tables  [B, max_blocks] int32, -1 padded
 *   context_lens  [B] int64; cu_seqlens_q [B+1] int32; positions [T] int64
 *   max_q_len     >= every cu_seqlens_q[b+1]-cu_seqlens_q[b] (host-known,
 *                 as the reference computes block_m from seqlens_q)
 *   kv_split_tokens  keys per workgroup split (multiple of 128); 0 = auto
 * Supported: D in {64, 128}; H % Hkv == 0; max_q_len <= 64; block_size a
 * power of two.  A kv head's rows ((H/Hkv) * max_q_len) beyond 64 are
 * served in launches over subsets of its query heads (the largest divisor
 * of H/Hkv whose rows fit), each re-reading the pair's K/V.
 * Workspace: nsv_verify_attention_workspace_size() bytes (0 when every
 * sequence fits one split): a 64 KiB area of per-(sequence, kv head)
 * arrival counters, then fp32 split partials.  The counter area must be
 * zero before a workspace's first call; every call leaves it zero (a
 * zero-filled allocation is enough).  Calls that share a workspace must not
 * run concurrently.  A call is one kernel (the key-split kernel merges its
 * splits itself), or two when the d-sliced kernel splits a sequence's keys
 * (the second merges the splits).
 */
size_t nsv_verify_attention_workspace_size(int B, int H, int Hkv, int D,
                                           int block_size, int max_blocks,
                                           int max_q_len, int dtype,
                                           int kv_split_tokens);
int nsv_verify_attention(void* out, const void* q, const void* k_cache,
                         const void* v_cache, const int32_t* block_tables,
                         const int64_t* context_lens,
                         const int32_t* cu_seqlens_q, const int64_t* positions,
                         float scale, int B, int T, int H, int Hkv, int D,
                         int block_size, int max_blocks, int max_q_len,
                         int dtype, int kv_split_tokens, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * Load-only measurement kernels, no reference counterpart (the ceilings
 * against which bench.py --ceiling reads the verify-attention kernels).
 * nsv_verify_attention_load_floor reads exactly the K/V bytes of a bf16,
 * D = 128 verify-attention call over `splits` key splits per (sequence, kv
 * head), in the key-split kernel's access pattern, and computes nothing;
 * nsv_stream_read reads `bytes` (a multiple of 16) of contiguous memory in
 * `workgroups` equal chunks.  `sink` is a device buffer of one uint32 per
 * workgroup that is written only for an improbable checksum.
 */
int nsv_verify_attention_load_floor(const void* k_cache, const void* v_cache,
                                    const int32_t* block_tables,
                                    const int64_t* context_lens, int B,
                                    int Hkv, int D, int block_size,
                                    int max_blocks, int splits, void* sink,
                                    void* stream);
int nsv_stream_read(const void* buf, size_t bytes, int workgroups,
                    void* sink, void* stream);

/*
 * Allocation-free variant of nsv_verify_attention: same arguments and
 * results, minus the workspace.  No reference counterpart: it is for callers
 * that cannot allocate device memory (code under hipGraph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Its scratch is a fixed
 * device array of nsv_verify_attention_noalloc_max_scratch() bytes (16 MiB)
 * inside the library, one per device, held until the process ends; a shape
 * whose nsv_verify_attention_workspace_size() exceeds it is rejected with
 * NSV_ERR_SCRATCH before anything is launched.  Never calls hipMalloc,
 * hipFree or an allocating library routine; the first call on a device
 * looks the array up and enqueues a clear of its counter area on `stream`.
 * Every call on a device shares that device's array: calls that overlap on
 * one GPU (concurrent streams, or host threads) race and must be ordered by
 * the caller, as calls sharing a workspace must be.
 */
size_t nsv_verify_attention_noalloc_max_scratch(void);
int nsv_verify_attention_noalloc(void* out, const void* q, const void* k_cache,
                                 const void* v_cache,
                                 const int32_t* block_tables,
                                 const int64_t* context_lens,
                                 const int32_t* cu_seqlens_q,
                                 const int64_t* positions, float scale, int B,
                                 int T, int H, int Hkv, int D, int block_size,
                                 int max_blocks, int max_q_len, int dtype,
                                 int kv_split_tokens, void* stream);

/* Timeline stamps of the verify-attention kernels, no reference
 * counterpart (a measurement aid).  Only a library built with NSV_STAMP=1
 * (libnaivspec_stamp.so) records them; the default library returns
 * NSV_ERR_UNSUPPORTED.  `buf` is device memory of calls * 4096 * 16 uint64
 * words: the i-th launch after this call writes, from thread 0 of each of
 * its workgroups w < 4096, the 100 MHz s_memrealtime clock at the kernel's
 * numbered points into words [(i % calls) * 4096 + w] * 16 + point, and the
 * XCD the workgroup ran on into word 15.  calls = 0 turns stamping off. */
int nsv_stamp_configure(void* buf, int calls);

/* The kernel nsv_verify_attention runs for these arguments on a device
 * with `cus` compute units (cus <= 0: the current device) and the key
 * splits per sequence it cuts (1: none).  Host-only query, launches
 * nothing; no reference counterpart (it exposes this library's plan for
 * tests and tuning).  Returns what nsv_verify_attention would return for
 * the shape (0, or the rejection code). */
#define NSV_ATTN_DSLICED 0   /* bf16, workgroup = (pair, head-dim slice) */
#define NSV_ATTN_KEY_SPLIT 1 /* bf16, workgroup = (pair, key split)      */
#define NSV_ATTN_F32 2       /* fp32, VALU dot products                  */
int nsv_verify_attention_plan(int B, int H, int Hkv, int D, int block_size,
                              int max_blocks, int max_q_len, int dtype,
                              int kv_split_tokens, int cus, int* kernel,
                              int* splits);

/*
 * Paged KV scatter.
 * Replaces layers/attention.py:71-112 (store_kvcache) and its kernel :9-68:
 *   k_cache[s / bs, s % bs, :, :] = key[t];  v_cache[...] = value[t]
 * for s = slot_mapping[t] >= 0; rows with slot -1 are skipped.
 *   key/value [T, Hkv, D]; caches [num_blocks, block_size, Hkv, D]
 */
int nsv_store_kv(const void* key, const void* value, void* k_cache,
                 void* v_cache, const int64_t* slot_mapping, int T, int Hkv,
                 int D, int block_size, int dtype, void* stream);

/*
 * Acceptance (greedy exact-match, and min(1, p_t/p_d) rejection sampling
 * with residual resampling), batched over B sequences with up to K drafts.
 * Replaces src/myvllm/spec_engine/rejection_sampler.py:24-98
 * (RejectionSampler.verify_greedy / verify_stochastic / verify) and the
 * engine's batched argmax + per-sequence walk (spec_llm_engine.py:224-247).
 *   target_logits  row r of sequence b at (b*target_seq_stride + r)*V,
 *                  rows 0..num_drafts[b] (the verify forward's K+1 rows;
 *                  graphed rounds pad each sequence to K+1 rows)
 *   drafts [B, K] int32, num_drafts [B] int32 (clamped to 0..K)
 *   out_tokens [B, K+1] int32: accepted drafts then the correction / bonus
 *   token; out_len [B] int32 in 1..num_drafts[b]+1
 * K <= 63.  Workspace: nsv_accept_workspace_size(B, K, V, dtype,
 * stochastic) bytes of per-chunk partial results; no initialisation
 * needed; calls that share a workspace must not run concurrently.  Greedy
 * acceptance is two kernels (chunk argmax, walk); stochastic acceptance
 * five (row statistics, accept walk, residual sums (only with draft rows),
 * samples, output tokens).  Argmax ties go to the lowest index and NaN
 * counts as the maximum, torch's rule.
 */
size_t nsv_accept_workspace_size(int B, int K, int V, int dtype, int stochastic);
int nsv_accept_greedy(const void* target_logits, int64_t target_seq_stride,
                      const int32_t* drafts, const int32_t* num_drafts, int B,
                      int K, int V, int dtype, int32_t* out_tokens,
                      int32_t* out_len, void* workspace,
                      size_t workspace_bytes, void* stream);
/*
 * Stochastic acceptance.  temperature [B] fp32: a sequence with
 * temperature <= 1e-6 is accepted greedily (rejection_sampler.py:95).
 * A sequence without draft rows (n-gram drafts, :75-85) samples every row
 * 0..num_drafts[b] and keeps drafts while they equal the samples, from
 * noise [K+1, V].  A sequence with draft rows (model drafts, :51-73) reads
 * draft row i at (b*draft_seq_stride + i*draft_row_stride)*V; uniforms
 * [B, K] fp32 decide u < min(1, p_t/p_d); one multinomial (the resample of
 * the first rejected row, or the bonus) uses noise [V].
 *   draft_logits NULL: no sequence has draft rows.
 *   draft_mode [B] (nullable): 0 marks a sequence without draft rows when
 *     draft_logits is given (a hybrid drafter's n-gram sequences,
 *     spec_engine/drafters.py:184-196); NULL: every sequence has them.
 *   noise: sequence b's noise at b*noise_seq_stride elements; 0 selects
 *     V when every sequence has draft rows, else (K+1)*V.
 * Randomness is input: torch.multinomial(p, 1) == argmax(p / q) for
 * q = Exp(1) draws in p's dtype (noise has the logits dtype), so a caller
 * drawing u = rand(K) and then q from the reference's generator reproduces
 * its samples.
 */
int nsv_accept_stochastic(const void* target_logits, int64_t target_seq_stride,
                          const void* draft_logits, int64_t draft_seq_stride,
                          int64_t draft_row_stride, const int32_t* draft_mode,
                          const int32_t* drafts, const int32_t* num_drafts,
                          const float* temperature, const float* uniforms,
                          const void* noise, int64_t noise_seq_stride, int B,
                          int K, int V, int dtype, int32_t* out_tokens,
                          int32_t* out_len, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * Token sampling of the decode / draft forward.
 * Replaces src/myvllm/layers/sampler.py:14-24 (SamplerLayer.forward): for
 * row b (at b*row_stride elements of logits, dtype), temperature[b] <= 1e-6
 * takes argmax(logits); otherwise argmax(softmax(logits / T) / q) with the
 * quotient and the softmax in fp32 (logits divided by an fp32 tensor
 * promote to fp32) and q = noise[b, :] fp32 [B, V], the reference's
 * exponential_(1).clamp_min_(1e-10) draws.  The token goes to
 * out_tokens[b*out_stride].  row_stride a multiple of V.  Workspace:
 * nsv_sample_workspace_size(); no initialisation needed.
 */
size_t nsv_sample_workspace_size(int B, int V, int dtype);
int nsv_sample(const void* logits, int64_t row_stride, const float* temperature,
               const float* noise, int B, int V, int dtype,
               int32_t* out_tokens, int64_t out_stride, void* workspace,
               size_t workspace_bytes, void* stream);

/*
 * N-gram (prompt-lookup) drafting on a device-resident token history.
 * Replaces src/myvllm/spec_engine/drafters.py:63-83 (NgramDrafter._lookup,
 * a bytes.rfind over the big-endian uint32 encoding of the history) and the
 * token choice of NgramDrafter.draft (:46-61), byte-exact including matches
 * at byte offsets inside a token.
 *   history [B, hist_stride] int32, hist_len [B]: tokens of each sequence
 *   out_drafts [B, K] int32, out_len [B] int32 (0: no match)
 * 1 <= min_n <= max_n <= 64, 1 <= K <= 64.
 */
int nsv_ngram_draft(const int32_t* history, const int32_t* hist_len,
                    int64_t hist_stride, int B, int min_n, int max_n, int K,
                    int32_t* out_drafts, int32_t* out_len, void* stream);

/*
 * Verify-row metadata from the device-resident round state.
 * Replaces the host row building of src/myvllm/engine/model_runner.py:
 * 734-774 (_run_spec_verify_graph).  For each sequence b with active[b]
 * and n = hist_len[b] > 0 tokens: rows b*(K+1) + j, j <= num_drafts[b],
 * get token history[b, n-1] (j = 0) or drafts[b, j-1], position n-1+j and
 * slot block_tables[b, pos / block_size] * block_size + pos % block_size;
 * remaining rows are inert pads (id 0, position -1, slot -1) and
 * context_lens[b] = n + num_drafts[b] (0 when inactive).  K + 1 <= 64.
 */
int nsv_prepare_verify(const int32_t* history, int64_t hist_stride,
                       const int32_t* hist_len, const int32_t* drafts,
                       const int32_t* num_drafts, const int32_t* block_tables,
                       int max_blocks, int block_size, const int32_t* active,
                       int B, int K, int64_t* input_ids, int64_t* positions,
                       int64_t* slot_mapping, int64_t* context_lens,
                       void* stream);

/*
 * Rows of a model drafter's K decode steps, all built in one launch.
 * Replaces the host staging of src/myvllm/engine/model_runner.py:784-823
 * (run_draft_steps_gpu).  For an active sequence b with n = hist_len[b]
 * confirmed tokens, step i feeds the token at position n-1+i (step 0: the
 * last confirmed token; step i > 0: the draft sampled by step i-1) and
 * attends keys 0..n-1+i:
 *   ids0/pos0/slot0 [2B]: step 0's rows, the tokens at n-2 and n-1 (the row
 *     at n-2 rewrites the draft-cache entry of a last draft that a fully
 *     accepted round never fed to the drafter; a pad when n < 2);
 *   positions/slot_mapping/context_lens [K, B] int64: step i's row at
 *     i*B + b (context n+i; row 0 of positions/slot_mapping is step 0's
 *     second row).
 * Inactive sequences get pads (id 0, position -1, slot -1, context 0).
 * (The reference passes context n+i+1, one key past the fed token;
 * positions past it hold no entry of this round, so this build uses n+i.)
 */
int nsv_prepare_draft(const int32_t* history, int64_t hist_stride,
                      const int32_t* hist_len, const int32_t* block_tables,
                      int max_blocks, int block_size, const int32_t* active,
                      int B, int K, int64_t* ids0, int64_t* pos0,
                      int64_t* slot0, int64_t* positions,
                      int64_t* slot_mapping, int64_t* context_lens,
                      void* stream);

/*
 * Commit of accepted tokens into the device-resident history.
 * Replaces src/myvllm/spec_engine/spec_llm_engine.py:249-291 (_commit):
 * appends at most max_tokens[b] - (hist_len[b] - prompt_len[b]) of the
 * num_tokens[b] accepted tokens, stopping after an eos token (unless
 * ignore_eos[b]) or when the length reaches max_len[b] (> 0); clears
 * active[b] when the sequence finishes (eos, max_tokens, max_len, or no
 * room in the history for another round) and writes the count appended
 * to committed[b].
 */
int nsv_commit(const int32_t* tokens, const int32_t* num_tokens,
               const int32_t* num_drafts, int32_t* history,
               int64_t hist_stride, int32_t* hist_len,
               const int32_t* prompt_len, const int32_t* max_tokens,
               const int32_t* max_len, const int32_t* ignore_eos, int eos,
               int32_t* active, int32_t* committed, int B, int K,
               void* stream);

/*
 * Fused elementwise stages of the Qwen3 verify forward (bf16 only).
 * nsv_rms_norm: out = rmsnorm(r) * weight with r = x + residual (or x when
 *   residual is NULL), r written to residual_out when not NULL; rows of E
 *   <= 4096.  Replaces layers/layernorm.py:18-35 (LayerNorm.forward with
 *   and without residual).
 * nsv_qk_norm_rope_store: the pre-attention epilogue over qkv
 *   [T, (H + 2*Hkv) * D]: per-head RMSNorm of q and k (q_norm_w, k_norm_w
 *   [D]), NeoX rotation at positions[t] from cos_sin [max_pos, D] (fp32,
 *   cos then sin), q written to q_out [T, H, D], k and v stored into the
 *   paged caches at slot_mapping[t] (slot < 0: not stored).  D even,
 *   <= 128.  positions == NULL: cos_sin holds one row per step row
 *   ([T, D], the table gathered at the rows' positions; max_pos >= T).
 *   Replaces models/qwen3.py:100-119 + layers/rotary_embedding.py:
 *   78-86 + layers/attention.py:71-112.
 * nsv_silu_mul: out [T, I] = silu(gate_up[:, :I]) * gate_up[:, I:].
 *   Replaces layers/activation.py:17-19.
 * nsv_embed_rms_norm: the forward's prologue: r = embed[ids[t]] (embed
 *   [vocab, E] bf16; an id outside [0, vocab) reads row 0, as the
 *   reference's single-GPU lookup does) written to
 *   residual_out, out = rmsnorm(r) * weight, and, when rope_out is not NULL,
 *   rope_out[t] = cos_sin[positions[t]] ([T, D] fp32; position < 0 takes
 *   row 0, past max_pos the last row), the per-row rotary table the
 *   epilogue takes with positions == NULL.  Replaces the embedding lookup
 *   (layers/embedding_head.py:32-46), layer 0's input LayerNorm
 *   (layers/layernorm.py:18-35) and the rotary cache lookup
 *   (layers/rotary_embedding.py:78-80).
 */
int nsv_rms_norm(const void* x, const void* residual, void* residual_out,
                 const void* weight, void* out, int T, int E, float eps,
                 void* stream);
int nsv_qk_norm_rope_store(const void* qkv, const void* q_norm_w,
                           const void* k_norm_w, const float* cos_sin,
                           int max_pos, const int64_t* positions,
                           const int64_t* slot_mapping, void* q_out,
                           void* k_cache, void* v_cache, int T, int H,
                           int Hkv, int D, float eps, void* stream);
int nsv_silu_mul(const void* gate_up, void* out, int T, int I, void* stream);
int nsv_embed_rms_norm(const int64_t* ids, const void* embed, int64_t vocab,
                       const void* weight, float eps, void* residual_out,
                       void* out, int T, int E, const int64_t* positions,
                       const float* cos_sin, int max_pos, int D,
                       float* rope_out, void* stream);

/*
 * Few-row bf16 linear layer of the verify forward: y = h W^T for the
 * M = B*(K+1) verify rows, W [N, K] row-major, fp32 accumulation, one bf16
 * rounding per output.  Replaces the F.linear projections of
 * src/myvllm/layers/linear.py (qkv_proj, o_proj, gate_up_proj, down_proj,
 * models/qwen3.py:74-151) and the LM head (layers/embedding_head.py:71-95),
 * and fuses their neighbours:
 *   norm_w != NULL: h = rmsnorm(x) * norm_w (layers/layernorm.py:18-35)
 *     with x the bf16 residual stream [M, K] and ss_in [nss_in, M] the
 *     partial sums of x^2 per row that a residual epilogue wrote (summed in
 *     a fixed order), evaluated as y = inv_rms(x) * (x W'^T) with
 *     W' = bf16(W * norm_w) (the norm weight folded into the weight rows);
 *     otherwise h = x.
 *   epilogue 0: y [M, N] = h W^T.
 *   epilogue 1 (SiluAndMul, layers/activation.py:17-19): W holds
 *     [gate; up] ([N = 2I, K]); y [M, I] = silu(gate) * up.
 *   epilogue 2 (the residual add of layernorm.py:29-31): resid [M, N] =
 *     bf16(h W^T) + resid, and ss_out [N/16, M] receives the partial sums
 *     of the new resid^2 over each 16-column tile; y is unused.
 * N % 16 == 0, K % 8 == 0.  For 32-80 rows and fewer than 128 column tiles
 * the reduction is split over up to 4 workgroups per tile, whose partials
 * meet in `workspace` (nsv_linear_workspace_size bytes: a fixed 64 KiB area
 * of per-tile arrival counters, then fp32 partials).  The counter area must
 * be zero before a workspace's first call; every call leaves it zero, so
 * one workspace serves every call of any shape on a stream (calls sharing
 * it must not run concurrently).  Otherwise no workspace is used.
 */
size_t nsv_linear_workspace_size(int M, int N, int K);
/* Rows of ss_out a residual-epilogue call with these M, N, K (and an
 * RMSNorm prologue or not) writes: one partial sum of r^2 per row for each
 * 16-column tile, or each 8-column tile where few rows over few tiles take
 * 8-column workgroups.  The consumer's nss_in. */
int nsv_linear_ss_rows(int M, int N, int K, int has_norm);
/* The dispatch nsv_linear takes for these arguments on a device with `cus`
 * compute units (cus <= 0: the current device): output columns per
 * workgroup (8, 16 or 32), workgroups per 16-column tile that split the
 * reduction (> 1 only with 16-column tiles), and whether half-size
 * reduction chunks are used (1), or 16-column tiles streamed whole by
 * single waves over activations staged in LDS (2: a plain projection with
 * at least 32 tiles per compute unit, K of 1024, 2048 or 4096 and
 * M (K + 8) bf16 within 160 KiB, such as the LM head).  Host-only query, launches nothing; no
 * reference counterpart (it exposes this library's tiling for tests and
 * tuning). */
int nsv_linear_plan(int M, int N, int K, int has_norm, int epilogue, int cus,
                    int* tile_cols, int* splits, int* half_chunks);
int nsv_linear(const void* x, const void* norm_w, const float* ss_in,
               int nss_in, float eps, const void* weight, void* y,
               void* resid, float* ss_out, int M, int N, int K,
               int epilogue, void* workspace, size_t workspace_bytes,
               void* stream);
/* nsv_linear for decode-shaped calls of at most 2 rows (a drafter's steps):
 * one wave per output column (per gate/up pair with epilogue 1), the whole
 * reduction in that wave, every load in one round trip, no workspace.  Same
 * operations per output as nsv_linear (W' = bf16(W * norm_w) with the
 * RMSNorm prologue, one bf16 rounding per product, the same epilogues); the
 * reduction order differs, so outputs may differ from nsv_linear's in the
 * last bf16 place.  K in {1024, 2048, 3072, 4096}; nss_in <= 256.  The
 * residual epilogue writes nsv_linear_decode_ss_rows(M, N) = N / 4 partial
 * sums per row (one per 4 columns), the nss_in of the consumer.  No
 * reference counterpart: the drafter's few-row path of this library's
 * forward (layers/linear.py's projections at one or two rows). */
int nsv_linear_decode(const void* x, const void* norm_w, const float* ss_in,
                      int nss_in, float eps, const void* weight, void* y,
                      void* resid, float* ss_out, int M, int N, int K,
                      int epilogue, void* stream);
int nsv_linear_decode_ss_rows(int M, int N);

/* The LM head (reference: src/myvllm/layers/embedding_head.py:71-83,
 * ParallelLMHead.forward's F.linear(x, weight) over the vocabulary rows) on
 * a weight repacked once at load time.  nsv_lm_head_pack writes the [N, K]
 * bf16 weight (N a multiple of 16, K of 1024, 2048 or 4096) into `packed`
 * (N * K bf16, a separate buffer) in the streaming kernel's load order: 16-byte
 * chunk ((t * K/256 + g) * 8 + s) * 64 + l holds row 16 t + (l % 16),
 * elements 256 g + 32 s + 8 (l / 16) .. + 7.  nsv_lm_head computes
 * y[M, N] = x[M, K] W^T from that copy (bf16, fp32 accumulation, the same
 * MFMA operands and order as nsv_linear's streaming dispatch, so the same
 * bits): each wave load reads 1 KiB in a row instead of half of 16 lines.
 * nsv_lm_head_rows gives the most rows it takes for this shape on the
 * current device (0: the shape is not one it streams); beyond that,
 * NSV_ERR_UNSUPPORTED (the caller then uses nsv_linear or a library GEMM
 * with the row-major weight).  The pack launches on `stream`; the head
 * launches nothing but its kernel and allocates nothing. */
int nsv_lm_head_rows(int N, int K);
int nsv_lm_head_pack(const void* weight, void* packed, int N, int K, void* stream);
int nsv_lm_head(const void* x, const void* packed, void* y, int M, int N, int K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NAIVSPEC_H */
