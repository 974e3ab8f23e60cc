"""The whole verification round on the device, one hipGraph per batch
bucket.

Per round and batch bucket B (K drafts, R = K + 1 rows per sequence):
  1. drafts, by the round's method:
       ngram  — prompt lookup on the device-resident history
                (spec_engine/drafters.py:46-83);
       model  — K decode steps of a draft model, each step's sampled token
                fed on the device to the next (drafters.py:116-154,
                engine/model_runner.py:784-847, layers/sampler.py:14-24);
       hybrid — n-gram first, the model's drafts for the sequences without a
                match (drafters.py:157-196);
  2. verify-row metadata: inputs [last_confirmed, d_1..d_K], positions,
     KV slots, context lengths (engine/model_runner.py:734-774);
  3. the target verify forward over B*R rows, logits of every row
     (models/qwen3.py, layers/attention.py:689-731);
  4. acceptance: greedy exact match, or (when the round is built
     stochastic) min(1, p_t/p_d) with residual resampling for model
     drafts and row sampling for n-gram drafts, per sequence, greedy for
     temperature <= 1e-6 (spec_llm_engine.py:224-247,
     rejection_sampler.py:24-98);
  5. commit of the accepted tokens into the history, with the caps of
     spec_llm_engine.py:249-291.
All of it runs on one stream from static buffers, random draws included
(torch's graph-safe generator), so the round is captured once per bucket
(the reference captures the verify forward and each draft step, :648-721,
:571-642, and does the rest in Python with host syncs).  The host reads one
small report per round.

Drafting for every sequence of a bucket: in a hybrid round the model
drafts all sequences and the n-gram result replaces it where there is a
match, which keeps the draft model's KV cache complete for every sequence
(the reference runs the model only for the sequences without a match, whose
draft caches then miss the tokens of n-gram rounds).

KV pages are reserved for a sequence's whole life at admission (prompt +
max_tokens + K + 1 positions), in the target's and the draft model's pools
alike (one block table serves both): with 288 GB of HBM the round never
needs the host to extend a block table.
"""

from __future__ import annotations

import torch

from naivllm_amd import _lib
from naivllm_amd.layers.qwen3 import Qwen3Verify
from naivllm_amd.spec_engine.drafters import ngram_draft
from naivllm_amd.spec_engine.rejection_sampler import accept_greedy, accept_stochastic, sample

DEFAULT_BUCKETS = (1, 2, 4, 8, 16, 32)
METHODS = ("ngram", "model", "hybrid", "none")


def prepare_verify(history, hist_len, drafts, num_drafts, block_tables, block_size, active, K, input_ids,
                   positions, slot_mapping, context_lens) -> None:
    B = hist_len.shape[0]
    rc = _lib.lib().nsv_prepare_verify(
        history.data_ptr(), history.stride(0), hist_len.data_ptr(), drafts.data_ptr(), num_drafts.data_ptr(),
        block_tables.data_ptr(), block_tables.shape[1], block_size, active.data_ptr(), B, K, input_ids.data_ptr(),
        positions.data_ptr(), slot_mapping.data_ptr(), context_lens.data_ptr(), _lib.stream_ptr(history.device))
    _lib.check(rc, "prepare_verify")


def prepare_draft(history, hist_len, block_tables, block_size, active, K, ids0, pos0, slot0, positions,
                  slot_mapping, context_lens) -> None:
    """Rows of the K draft steps (positions/slot_mapping/context_lens are
    flat [K*B] buffers, step i at i*B)."""
    B = hist_len.shape[0]
    rc = _lib.lib().nsv_prepare_draft(
        history.data_ptr(), history.stride(0), hist_len.data_ptr(), block_tables.data_ptr(), block_tables.shape[1],
        block_size, active.data_ptr(), B, K, ids0.data_ptr(), pos0.data_ptr(), slot0.data_ptr(),
        positions.data_ptr(), slot_mapping.data_ptr(), context_lens.data_ptr(), _lib.stream_ptr(history.device))
    _lib.check(rc, "prepare_draft")


def commit(tokens, num_tokens, num_drafts, history, hist_len, prompt_len, max_tokens, max_len, ignore_eos, eos,
           active, committed, K) -> None:
    B = hist_len.shape[0]
    rc = _lib.lib().nsv_commit(
        tokens.data_ptr(), num_tokens.data_ptr(), num_drafts.data_ptr(), history.data_ptr(), history.stride(0),
        hist_len.data_ptr(), prompt_len.data_ptr(), max_tokens.data_ptr(), max_len.data_ptr(), ignore_eos.data_ptr(),
        eos, active.data_ptr(), committed.data_ptr(), B, K, _lib.stream_ptr(history.device))
    _lib.check(rc, "commit")


class VerifyRound:
    def __init__(self, model: Qwen3Verify, max_batch: int, num_spec_tokens: int, min_ngram: int, max_ngram: int,
                 history_len: int, max_blocks: int, eos_token_id: int = -1, method: str = "ngram",
                 draft_model: Qwen3Verify | None = None, stochastic: bool = False, buckets=DEFAULT_BUCKETS):
        if method not in METHODS:
            raise ValueError(f"unknown round method {method!r}; expected one of {METHODS}")
        if method in ("model", "hybrid"):
            if draft_model is None:
                raise ValueError(f"a {method} round needs a draft model")
            if draft_model.cfg.vocab_size != model.cfg.vocab_size:
                raise ValueError("draft and target models must share the vocabulary")
            if num_spec_tokens < 1:
                raise ValueError("a model drafter needs num_spec_tokens >= 1")
        dev = model.device
        self.model = model
        self.draft_model = draft_model if method in ("model", "hybrid") else None
        self.method = method
        self.K = num_spec_tokens if method != "none" else 0
        self.R = self.K + 1
        self.min_n, self.max_n = min_ngram, max_ngram
        self.eos = eos_token_id
        self.max_batch = max_batch
        self.buckets = sorted({b for b in buckets if b <= max_batch} | {max_batch})
        self.stochastic = stochastic
        K, R, V = self.K, self.R, model.cfg.vocab_size
        i32 = dict(dtype=torch.int32, device=dev)
        i64 = dict(dtype=torch.int64, device=dev)
        rows = max_batch * R
        self.history = torch.zeros(max_batch, history_len, **i32)
        self.hist_len = torch.zeros(max_batch, **i32)
        self.prompt_len = torch.zeros(max_batch, **i32)
        self.max_tokens = torch.zeros(max_batch, **i32)
        self.max_len = torch.zeros(max_batch, **i32)
        self.ignore_eos = torch.zeros(max_batch, **i32)
        # the round's report rows, read back by the host in one transfer: active
        # flags, tokens committed, tokens drafted, drafts from the model.  The
        # per-sequence state below is these rows themselves (no copies per round).
        self.report_dev = torch.zeros(4, max_batch, **i32)
        self.active = self.report_dev[0]
        self.temperature = torch.zeros(max_batch, dtype=torch.float32, device=dev)
        self.block_tables = torch.full((max_batch, max_blocks), -1, **i32)
        self.drafts = torch.zeros(max_batch, max(K, 1), **i32)
        self.num_drafts = self.report_dev[2]
        self.draft_mode = self.report_dev[3]  # 1: the sequence's drafts came from the model
        self.input_ids = torch.zeros(rows, **i64)
        self.positions = torch.full((rows,), -1, **i64)
        self.slot_mapping = torch.full((rows,), -1, **i64)
        self.context_lens = torch.zeros(max_batch, **i64)
        self.logits = torch.empty(rows, V, dtype=model.dtype, device=dev)
        self.out_tokens = torch.zeros(max_batch, R, **i32)
        self.out_len = torch.zeros(max_batch, **i32)
        self.committed = self.report_dev[1]
        self.cu = {b: torch.arange(0, b * R + 1, R, **i32) for b in self.buckets}
        if method == "hybrid":
            self.ng_drafts = torch.zeros(max_batch, K, **i32)
            self.ng_len = torch.zeros(max_batch, **i32)
        if self.draft_model is not None:
            self.model_drafts = torch.zeros(max_batch, K, **i32)
            self.full_k = torch.full((max_batch,), K, **i32)
            self.ids0 = torch.zeros(2 * max_batch, **i64)
            self.pos0 = torch.full((2 * max_batch,), -1, **i64)
            self.slot0 = torch.full((2 * max_batch,), -1, **i64)
            self.dpos = torch.full((K * max_batch,), -1, **i64)
            self.dslot = torch.full((K * max_batch,), -1, **i64)
            self.dctx = torch.zeros(K * max_batch, **i64)
            self.step0_logits = torch.empty(2 * max_batch, V, dtype=model.dtype, device=dev)
            self.draft_logits = torch.empty(K, max_batch, V, dtype=model.dtype, device=dev)  # step i, sequence b
            self.draft_noise = torch.ones(K, max_batch, V, dtype=torch.float32, device=dev)
            self.cu1 = {b: torch.arange(0, b + 1, **i32) for b in self.buckets}
            self.cu2 = {b: torch.arange(0, 2 * b + 1, 2, **i32) for b in self.buckets}
        if stochastic:
            self.uniforms = torch.zeros(max_batch, max(K, 1), dtype=torch.float32, device=dev)
            per_seq = (V,) if method == "model" else (R, V)  # model drafts only: one multinomial per sequence
            self.accept_noise = torch.ones(max_batch, *per_seq, dtype=model.dtype, device=dev)
        # two host copies of the report, so that one round's report can be read
        # while the next round runs (launch / collect)
        self.reports = [torch.zeros(4, max_batch, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self.report_ready = [torch.cuda.Event() for _ in range(2)]
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}

    def bucket_for(self, n: int) -> int:
        return min(b for b in self.buckets if b >= n)

    def _cu_rows(self, table: dict, B: int, step: int) -> torch.Tensor:
        """cu_seqlens of B sequences of `step` rows each (built ahead for the
        buckets; an eager call with another B builds its own)."""
        t = table.get(B)
        if t is None:
            t = table[B] = torch.arange(0, B * step + 1, step, dtype=torch.int32, device=self.model.device)
        return t

    # ------------------------------------------------------------- drafting
    def _model_draft(self, B: int) -> None:
        """K decode steps of the draft model for slots 0..B-1: step 0 feeds
        the last two confirmed tokens (2 rows per sequence), step i > 0 the
        token sampled by step i-1; every step's logits row is kept for the
        acceptance and its sample becomes the draft."""
        dm, K = self.draft_model, self.K
        prepare_draft(self.history[:B], self.hist_len[:B], self.block_tables[:B], dm.block_size, self.active[:B], K,
                      self.ids0[:2 * B], self.pos0[:2 * B], self.slot0[:2 * B], self.dpos[:K * B],
                      self.dslot[:K * B], self.dctx[:K * B])
        if self.stochastic:
            self.draft_noise[:, :B].exponential_(1).clamp_min_(1e-10)  # layers/sampler.py:23
        for i in range(K):
            if i == 0:
                dm.forward(self.ids0[:2 * B], self.pos0[:2 * B], self.slot0[:2 * B], self.block_tables[:B],
                           self.dctx[:B], self._cu_rows(self.cu2, B, 2), 2, logits_out=self.step0_logits[:2 * B])
                self.draft_logits[0, :B].copy_(self.step0_logits[1:2 * B:2])
            else:
                s = slice(i * B, (i + 1) * B)
                dm.forward(self.model_drafts[:B, i - 1], self.dpos[s], self.dslot[s], self.block_tables[:B],
                           self.dctx[s], self._cu_rows(self.cu1, B, 1), 1, logits_out=self.draft_logits[i, :B])
            sample(self.draft_logits[i, :B], self.temperature[:B], self.draft_noise[i, :B],
                   out=self.model_drafts[:B, i])

    def _draft(self, B: int) -> None:
        K = self.K
        if self.method == "none" or K == 0:
            self.num_drafts[:B].zero_()
            return
        if self.method == "ngram":
            ngram_draft(self.history[:B], self.hist_len[:B], K, self.min_n, self.max_n,
                        out_drafts=self.drafts[:B, :K], out_len=self.num_drafts[:B])
            return
        self._model_draft(B)
        if self.method == "model":
            self.drafts[:B, :K].copy_(self.model_drafts[:B])
            self.num_drafts[:B].copy_(self.full_k[:B])
            self.draft_mode[:B].fill_(1)
            return
        # hybrid: the n-gram continuation where the history has a match, else the model's drafts
        ngram_draft(self.history[:B], self.hist_len[:B], K, self.min_n, self.max_n,
                    out_drafts=self.ng_drafts[:B], out_len=self.ng_len[:B])
        use_ng = self.ng_len[:B] > 0
        torch.where(use_ng[:, None], self.ng_drafts[:B], self.model_drafts[:B], out=self.drafts[:B, :K])
        torch.where(use_ng, self.ng_len[:B], self.full_k[:B], out=self.num_drafts[:B])
        torch.logical_not(use_ng, out=self.draft_mode[:B])

    # ---------------------------------------------------------------- round
    def body(self, B: int) -> None:
        """One round for slots 0..B-1 (all device work, on the current stream)."""
        K, R = self.K, self.R
        rows = B * R
        self._draft(B)
        prepare_verify(self.history[:B], self.hist_len[:B], self.drafts[:B, :K], self.num_drafts[:B],
                       self.block_tables[:B], self.model.block_size, self.active[:B], K, self.input_ids[:rows],
                       self.positions[:rows], self.slot_mapping[:rows], self.context_lens[:B])
        self.model.forward(self.input_ids[:rows], self.positions[:rows], self.slot_mapping[:rows],
                           self.block_tables[:B], self.context_lens[:B], self._cu_rows(self.cu, B, R), R,
                           logits_out=self.logits[:rows])
        if self.stochastic:
            self.uniforms[:B].uniform_()
            self.accept_noise[:B].exponential_(1)
            with_rows = self.draft_model is not None
            accept_stochastic(self.logits[:rows], self.drafts[:B, :K], self.num_drafts[:B], self.temperature[:B],
                              self.accept_noise[:B], uniforms=self.uniforms[:B, :K] if with_rows else None,
                              draft_logits=self.draft_logits if with_rows else None, target_seq_stride=R,
                              draft_seq_stride=1, draft_row_stride=self.max_batch,
                              draft_mode=self.draft_mode[:B] if self.method == "hybrid" else None,
                              out_tokens=self.out_tokens[:B], out_len=self.out_len[:B])
        else:
            accept_greedy(self.logits[:rows], self.drafts[:B, :K], self.num_drafts[:B], R,
                          out_tokens=self.out_tokens[:B], out_len=self.out_len[:B])
        commit(self.out_tokens[:B], self.out_len[:B], self.num_drafts[:B], self.history[:B], self.hist_len[:B],
               self.prompt_len[:B], self.max_tokens[:B], self.max_len[:B], self.ignore_eos[:B], self.eos,
               self.active[:B], self.committed[:B], K)
        # (the report rows are the state itself: the caller copies report_dev to the host)

    def capture(self) -> None:
        """Capture one graph per bucket (largest first, each in its own
        memory pool as the reference's verify graphs, model_runner.py:
        672-675).  Runs every bucket once eagerly first with every slot
        inactive, so workspaces reach their final size outside capture and
        the warm-up commits nothing."""
        saved = self.active.clone()
        self.active.zero_()
        self.graphs = {}
        for b in sorted(self.buckets, reverse=True):
            self.body(b)
        torch.cuda.synchronize(self.model.device)
        for b in sorted(self.buckets, reverse=True):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.body(b)
            self.graphs[b] = g
        torch.cuda.synchronize(self.model.device)
        self.active.copy_(saved)

    def launch(self, B: int, slot: int = 0) -> None:
        """Enqueue one round over slots 0..B-1 (B a bucket) and the copy of
        its report into host buffer `slot` (0 or 1); returns at once."""
        g = self.graphs.get(B)
        if g is not None:
            g.replay()
        else:
            self.body(B)
        # the whole [4, max_batch] block: one contiguous transfer (a column slice
        # would first be gathered by a device copy kernel)
        self.reports[slot].copy_(self.report_dev, non_blocking=True)
        self.report_ready[slot].record(torch.cuda.current_stream(self.model.device))

    def collect(self, B: int, slot: int = 0) -> torch.Tensor:
        """Wait for the report launched into `slot`; returns it as [4, B]:
        active flags, tokens committed, tokens drafted, model-draft flags."""
        self.report_ready[slot].synchronize()
        return self.reports[slot][:, :B]

    def run(self, B: int) -> torch.Tensor:
        """One round over slots 0..B-1, waited for; returns its report [4, B]."""
        self.launch(B, 0)
        return self.collect(B, 0)
