"""The whole greedy n-gram verification round on the device, one hipGraph
per batch bucket.

Per round and batch bucket B (K drafts, R = K + 1 rows per sequence):
  1. n-gram drafts from the device-resident history
     (spec_engine/drafters.py:46-83);
  2. verify-row metadata: inputs [last_confirmed, d_1..d_K], positions,
     KV slots, context lengths (engine/model_runner.py:734-774);
  3. the Qwen3 verify forward over B*R rows, logits of every row
     (models/qwen3.py, layers/attention.py:689-731);
  4. greedy acceptance (spec_llm_engine.py:224-243, rejection_sampler.py:
     25-36);
  5. commit of the accepted tokens into the history, with the caps of
     spec_llm_engine.py:249-291.
All five run on one stream from static buffers, so the round is captured
once per bucket (the reference captures only step 3, :648-721, and does
steps 1, 2, 4 and 5 in Python with a host sync).  The host reads one small
report per round (active flags, committed and drafted counts).

KV pages are reserved for a sequence's whole life at admission (prompt +
max_tokens + K + 1 positions): with 288 GB of HBM the round never needs the
host to extend a block table.
"""

from __future__ import annotations

import torch

from naivllm_amd import _lib
from naivllm_amd.layers.qwen3 import Qwen3Verify
from naivllm_amd.spec_engine.drafters import ngram_draft
from naivllm_amd.spec_engine.rejection_sampler import accept_greedy

DEFAULT_BUCKETS = (1, 2, 4, 8, 16, 32)


def prepare_verify(history, hist_len, drafts, num_drafts, block_tables, block_size, active, K, input_ids,
                   positions, slot_mapping, context_lens) -> None:
    B = hist_len.shape[0]
    rc = _lib.lib().nsv_prepare_verify(
        history.data_ptr(), history.stride(0), hist_len.data_ptr(), drafts.data_ptr(), num_drafts.data_ptr(),
        block_tables.data_ptr(), block_tables.shape[1], block_size, active.data_ptr(), B, K, input_ids.data_ptr(),
        positions.data_ptr(), slot_mapping.data_ptr(), context_lens.data_ptr(), _lib.stream_ptr(history.device))
    _lib.check(rc, "prepare_verify")


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
                 history_len: int, max_blocks: int, eos_token_id: int = -1, draft: bool = True,
                 buckets=DEFAULT_BUCKETS):
        dev = model.device
        self.model = model
        self.K = num_spec_tokens
        self.R = self.K + 1
        self.min_n, self.max_n = min_ngram, max_ngram
        self.eos = eos_token_id
        self.draft = draft
        self.max_batch = max_batch
        self.buckets = sorted({b for b in buckets if b <= max_batch} | {max_batch})
        i32 = dict(dtype=torch.int32, device=dev)
        i64 = dict(dtype=torch.int64, device=dev)
        rows = max_batch * self.R
        self.history = torch.zeros(max_batch, history_len, **i32)
        self.hist_len = torch.zeros(max_batch, **i32)
        self.prompt_len = torch.zeros(max_batch, **i32)
        self.max_tokens = torch.zeros(max_batch, **i32)
        self.max_len = torch.zeros(max_batch, **i32)
        self.ignore_eos = torch.zeros(max_batch, **i32)
        self.active = torch.zeros(max_batch, **i32)
        self.block_tables = torch.full((max_batch, max_blocks), -1, **i32)
        self.drafts = torch.zeros(max_batch, max(self.K, 1), **i32)
        self.num_drafts = torch.zeros(max_batch, **i32)
        self.input_ids = torch.zeros(rows, **i64)
        self.positions = torch.full((rows,), -1, **i64)
        self.slot_mapping = torch.full((rows,), -1, **i64)
        self.context_lens = torch.zeros(max_batch, **i64)
        self.logits = torch.empty(rows, model.cfg.vocab_size, dtype=model.dtype, device=dev)
        self.out_tokens = torch.zeros(max_batch, self.R, **i32)
        self.out_len = torch.zeros(max_batch, **i32)
        self.committed = torch.zeros(max_batch, **i32)
        self.cu = {b: torch.arange(0, b * self.R + 1, self.R, **i32) for b in self.buckets}
        self.report_dev = torch.zeros(3, max_batch, **i32)
        self.report = torch.zeros(3, max_batch, dtype=torch.int32, pin_memory=True)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}

    def bucket_for(self, n: int) -> int:
        return min(b for b in self.buckets if b >= n)

    def body(self, B: int) -> None:
        """One round for slots 0..B-1 (all device work, on the current stream)."""
        K, R = self.K, self.R
        rows = B * R
        if self.draft and K > 0:
            ngram_draft(self.history[:B], self.hist_len[:B], K, self.min_n, self.max_n,
                        out_drafts=self.drafts[:B, :K], out_len=self.num_drafts[:B])
        prepare_verify(self.history[:B], self.hist_len[:B], self.drafts[:B, :K], self.num_drafts[:B],
                       self.block_tables[:B], self.model.block_size, self.active[:B], K, self.input_ids[:rows],
                       self.positions[:rows], self.slot_mapping[:rows], self.context_lens[:B])
        self.model.forward(self.input_ids[:rows], self.positions[:rows], self.slot_mapping[:rows],
                           self.block_tables[:B], self.context_lens[:B], self.cu[B], R,
                           logits_out=self.logits[:rows])
        accept_greedy(self.logits[:rows], self.drafts[:B, :K], self.num_drafts[:B], R,
                      out_tokens=self.out_tokens[:B], out_len=self.out_len[:B])
        commit(self.out_tokens[:B], self.out_len[:B], self.num_drafts[:B], self.history[:B], self.hist_len[:B],
               self.prompt_len[:B], self.max_tokens[:B], self.max_len[:B], self.ignore_eos[:B], self.eos,
               self.active[:B], self.committed[:B], K)
        # the round's report, copied to the host by the caller in one transfer
        self.report_dev[0, :B].copy_(self.active[:B])
        self.report_dev[1, :B].copy_(self.committed[:B])
        self.report_dev[2, :B].copy_(self.num_drafts[:B])

    def capture(self) -> None:
        """Capture one graph per bucket (largest first, each in its own
        memory pool as the reference's verify graphs, model_runner.py:
        672-675).  Runs every bucket once eagerly first with every slot
        inactive, so workspaces reach their final size outside capture and
        the warm-up commits nothing."""
        saved = self.active.clone()
        self.active.zero_()
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

    def run(self, B: int) -> torch.Tensor:
        """One round over slots 0..B-1 (B a bucket); returns the host report
        [3, B]: active flags, tokens committed, tokens drafted."""
        g = self.graphs.get(B)
        if g is not None:
            g.replay()
        else:
            self.body(B)
        self.report[:, :B].copy_(self.report_dev[:, :B], non_blocking=True)
        torch.cuda.current_stream(self.model.device).synchronize()
        return self.report[:, :B]
