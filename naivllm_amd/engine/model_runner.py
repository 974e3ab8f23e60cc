"""The verification surface of the reference's ModelRunner.

Drop-in for ``ModelRunner.prepare_spec_verify`` / ``run_spec_verify`` /
``capture_verify_graphs`` and ``verify_vars`` (src/myvllm/engine/
model_runner.py:443-483, :648-721, :724-777): host ``Sequence`` objects
whose drafts were appended by a drafter (``seq.draft_tokens``) go in; the
target's logits for rows [last_confirmed, d_1 .. d_K_i] of every sequence
come out.  Graphed (the default) the rows of sequence i start at
i * (K + 1), padded to K + 1 rows with inert rows (token 0, position -1,
slot -1), and the result is a view of ``verify_vars["logits"]``, valid
until the next call; eager the rows are packed back to back.  The K/V of
the verified rows land in the model's paged cache at the sequences' slots
(the caller has extended their block tables, e.g. with
``BlockManager.ensure_capacity``).

The forward is the library's Qwen3 verify forward (layers.qwen3); one
hipGraph per batch bucket {1, 2, 4, 8, ...} is captured with static
buffers, as the reference captures its verify graphs.
"""

from __future__ import annotations

import torch

from naivllm_amd.layers.qwen3 import Qwen3Verify
from naivllm_amd.utils.context import get_context, reset_context, set_context

BUCKETS = (1, 2, 4, 8, 16, 32)


class ModelRunner:
    def __init__(self, model: Qwen3Verify, max_num_sequences: int, num_spec_tokens: int, max_model_length: int,
                 table_attr: str = "block_table", enforce_eager: bool = False):
        if model.block_size <= 0:
            raise ValueError("allocate the model's KV cache before building its runner")
        self.model = model
        self.block_size = model.block_size
        self.table_attr = table_attr
        self.max_num_sequences = max_num_sequences
        k = num_spec_tokens
        dev = model.device
        rows = max_num_sequences * (k + 1)
        max_blocks = -(-(max_model_length + k + 1) // self.block_size)
        i64 = dict(dtype=torch.int64, device=dev)
        self.verify_vars = {
            "k": k,
            "input_ids": torch.zeros(rows, **i64),
            "slot_mapping": torch.full((rows,), -1, **i64),
            "positions": torch.full((rows,), -1, **i64),
            "context_lens": torch.zeros(max_num_sequences, **i64),
            "block_tables": torch.full((max_num_sequences, max_blocks), -1, dtype=torch.int32, device=dev),
            "logits": torch.empty(rows, model.cfg.vocab_size, dtype=model.dtype, device=dev),
        }
        self.buckets = sorted({b for b in BUCKETS if b <= max_num_sequences} | {max_num_sequences})
        self._cu = {b: torch.arange(0, b * (k + 1) + 1, k + 1, dtype=torch.int32, device=dev) for b in self.buckets}
        self.verify_graphs: dict[int, torch.cuda.CUDAGraph] = {}
        if not enforce_eager:
            self.capture_verify_graphs()

    def _table(self, seq) -> list[int]:
        return getattr(seq, self.table_attr)

    def _rows(self, seq) -> tuple[list[int], list[int], list[int]]:
        """Token ids, positions and slots of the sequence's verify rows:
        positions n-1 .. len(seq)-1 with n = len(seq) - len(draft_tokens)."""
        table = self._table(seq)
        n = len(seq) - len(seq.draft_tokens)
        pos = list(range(n - 1, len(seq)))
        return ([seq.token_ids[p] for p in pos], pos,
                [table[p // self.block_size] * self.block_size + p % self.block_size for p in pos])

    # ------------------------------------------------------------------ eager
    def prepare_spec_verify(self, seqs) -> torch.Tensor:
        """Packed rows of ``seqs`` (model_runner.py:443-483): publishes the
        step's metadata with ``set_context`` (is_prefill and is_verify set,
        cu_seqlens_q, max_seqlen_q/k, slot_mapping, context_lens,
        block_tables -1 padded, seqlens_q/k, positions) for the layers to
        read, and returns the rows' input_ids, all on the model's device."""
        ids, pos, slots, cu, qlens = [], [], [], [0], []
        for seq in seqs:
            a, b, c = self._rows(seq)
            ids += a
            pos += b
            slots += c
            cu.append(cu[-1] + len(a))
            qlens.append(len(a))
        width = max(len(self._table(s)) for s in seqs)
        bt = [self._table(s) + [-1] * (width - len(self._table(s))) for s in seqs]
        klens = [len(s) for s in seqs]
        dev = self.model.device
        t = lambda x, dt: torch.tensor(x, dtype=dt, device=dev)  # noqa: E731
        set_context(True, is_verify=True, cu_seqlens_q=t(cu, torch.int32), cu_seqlens_k=None,
                    max_seqlen_q=max(qlens), max_seqlen_k=max(klens), slot_mapping=t(slots, torch.int64),
                    context_lens=t(klens, torch.int64), block_tables=t(bt, torch.int32), seqlens_q=qlens,
                    seqlens_k=klens, positions=t(pos, torch.int64))
        return t(ids, torch.int64)

    # ---------------------------------------------------------------- graphed
    def _forward_bucket(self, B: int) -> None:
        v = self.verify_vars
        rows = B * (v["k"] + 1)
        self.model.forward(v["input_ids"][:rows], v["positions"][:rows], v["slot_mapping"][:rows],
                           v["block_tables"][:B], v["context_lens"][:B], self._cu[B], v["k"] + 1,
                           logits_out=v["logits"][:rows])

    def capture_verify_graphs(self) -> None:
        """One graph per bucket, captured from inert rows (no KV is written)."""
        v = self.verify_vars
        v["slot_mapping"].fill_(-1)
        v["positions"].fill_(-1)
        v["context_lens"].zero_()
        v["block_tables"].fill_(-1)
        for b in sorted(self.buckets, reverse=True):
            self._forward_bucket(b)  # workspaces reach their final size outside capture
        torch.cuda.synchronize(self.model.device)
        self.verify_graphs = {}
        for b in sorted(self.buckets, reverse=True):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._forward_bucket(b)
            self.verify_graphs[b] = g
        torch.cuda.synchronize(self.model.device)

    @torch.inference_mode()
    def run_spec_verify(self, seqs) -> torch.Tensor:
        """Logits of every sequence's verify rows: graphed, [B_bucket * (K+1),
        vocab] with sequence i's rows at i * (K + 1) (a view of
        verify_vars["logits"]); eager, the packed rows."""
        if not seqs:
            raise ValueError("no sequences to verify")
        if not self.verify_graphs:
            ids = self.prepare_spec_verify(seqs)
            c = get_context()
            try:
                return self.model.forward(ids, c.positions, c.slot_mapping, c.block_tables, c.context_lens,
                                          c.cu_seqlens_q, c.max_seqlen_q)
            finally:
                reset_context()
        v = self.verify_vars
        k = v["k"]
        if len(seqs) > self.max_num_sequences:
            raise ValueError(f"{len(seqs)} sequences exceed the runner's {self.max_num_sequences}")
        if any(len(s.draft_tokens) > k for s in seqs):
            raise ValueError(f"a sequence carries more than K = {k} drafts")
        B = min(b for b in self.verify_graphs if b >= len(seqs))
        ids, pos, slots = [0] * (B * (k + 1)), [-1] * (B * (k + 1)), [-1] * (B * (k + 1))
        ctx = [0] * B
        width = v["block_tables"].shape[1]
        bt = [[-1] * width for _ in range(B)]
        for i, seq in enumerate(seqs):
            a, b, c = self._rows(seq)
            r0 = i * (k + 1)
            ids[r0:r0 + len(a)], pos[r0:r0 + len(b)], slots[r0:r0 + len(c)] = a, b, c
            ctx[i] = len(seq)
            table = self._table(seq)
            if len(table) > width:
                raise ValueError("block table longer than the runner's max_model_length allows")
            bt[i][:len(table)] = table
        rows = B * (k + 1)
        v["input_ids"][:rows].copy_(torch.tensor(ids, dtype=torch.int64))
        v["positions"][:rows].copy_(torch.tensor(pos, dtype=torch.int64))
        v["slot_mapping"][:rows].copy_(torch.tensor(slots, dtype=torch.int64))
        v["context_lens"][:B].copy_(torch.tensor(ctx, dtype=torch.int64))
        v["block_tables"][:B].copy_(torch.tensor(bt, dtype=torch.int32))
        self.verify_graphs[B].replay()
        return v["logits"][:rows]
