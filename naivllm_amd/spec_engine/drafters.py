"""Token drafters on the GPU.

The reference's drafter protocol (src/myvllm/spec_engine/drafters.py):
``draft(seqs)`` appends each sequence's drafts with ``append_token``,
records them in ``seq.draft_tokens`` and returns ``(drafts, rows)`` with
the draft distributions (``None`` for n-gram drafts); ``prefill`` and
``can_draft`` are optional hooks.

``NgramDrafter`` (:26-83): the lookup (``_lookup``, a ``bytes.rfind`` over
the big-endian uint32 encoding of the history) runs as one GPU kernel over
the whole batch; ``draft_device`` is the device-resident form the
verification round uses on a history that never leaves the GPU.

``ModelDrafter`` (:86-154) runs K decode steps of a draft model
(``DraftRunner``, the reference's draft ModelRunner with its own paged KV
cache and ``draft_block_table``), each step's token sampled on the device
(layers/sampler.py) and fed to the next step without a host round trip;
the host synchronises once per call.  ``HybridDrafter`` (:157-196): n-gram
first, the model for the sequences without a match.
"""

from __future__ import annotations

import torch

from naivllm_amd import _lib


def ngram_draft(history: torch.Tensor, hist_len: torch.Tensor, k: int, min_n: int, max_n: int,
                out_drafts: torch.Tensor | None = None,
                out_len: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """history [B, S] int32 on the GPU (row b holds hist_len[b] tokens).
    Returns (drafts [B, k] int32, lengths [B] int32) on the device."""
    if not history.is_cuda or history.dtype != torch.int32 or history.dim() != 2 or history.stride(1) != 1:
        raise ValueError("history must be a (batch, length) int32 GPU tensor with contiguous rows")
    B = history.shape[0]
    dev = history.device
    hist_len = hist_len.to(device=dev, dtype=torch.int32).contiguous()
    if hist_len.numel() != B:
        raise ValueError("hist_len must hold one length per sequence")
    if out_drafts is None:
        out_drafts = torch.empty(B, k, dtype=torch.int32, device=dev)
    if out_len is None:
        out_len = torch.empty(B, dtype=torch.int32, device=dev)
    rc = _lib.lib().nsv_ngram_draft(history.data_ptr(), hist_len.data_ptr(), history.stride(0), B, min_n, max_n, k,
                                    out_drafts.data_ptr(), out_len.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(rc, "ngram_draft")
    return out_drafts, out_len


class NgramDrafter:
    """Prompt-lookup drafting (drafters.py:26-61): for n from
    ``max_ngram_size`` down to ``min_ngram_size``, the continuation of the
    most recent earlier occurrence of the history's last n tokens."""

    name = "ngram"

    def __init__(self, num_speculative_tokens: int = 5, min_ngram_size: int = 2, max_ngram_size: int = 8,
                 device: torch.device | str | None = None):
        self.num_speculative_tokens = num_speculative_tokens
        self.min_ngram_size = min_ngram_size
        self.max_ngram_size = max_ngram_size
        self.device = torch.device(device) if device is not None else None

    def _device(self) -> torch.device:
        return self.device if self.device is not None else torch.device("cuda", torch.cuda.current_device())

    def draft_device(self, history: torch.Tensor, hist_len: torch.Tensor, out_drafts=None, out_len=None):
        return ngram_draft(history, hist_len, self.num_speculative_tokens, self.min_ngram_size,
                           self.max_ngram_size, out_drafts, out_len)

    def draft(self, seqs) -> tuple[list[list[int]], list]:
        """Append drafted tokens onto each sequence (the engine rolls them
        back after verification); returns (draft_lists, [None] * B)."""
        if not seqs:
            return [], []
        dev = self._device()
        S = max(1, max(len(s.token_ids) for s in seqs))
        host = torch.zeros(len(seqs), S, dtype=torch.int32, pin_memory=True)
        for b, s in enumerate(seqs):
            if s.token_ids:
                host[b, :len(s.token_ids)] = torch.as_tensor(s.token_ids, dtype=torch.int32)
        lens = torch.tensor([len(s.token_ids) for s in seqs], dtype=torch.int32, pin_memory=True)
        drafts, n = self.draft_device(host.to(dev, non_blocking=True), lens.to(dev, non_blocking=True))
        drafts, n = drafts.cpu().tolist(), n.cpu().tolist()
        out = []
        for s, d, k in zip(seqs, drafts, n):
            drafted = d[:k]
            s.draft_tokens = list(drafted)
            for t in drafted:
                s.append_token(t)
            out.append(drafted)
        return out, [None] * len(seqs)


class DraftRunner:
    """A draft model with its own paged KV pool, addressed through
    ``seq.draft_block_table`` (the reference's draft ModelRunner,
    spec_llm_engine.py:104-137, model_runner.py:784-847).  Eager: the
    device round (engine/verify_round.py) is the graph-captured form."""

    def __init__(self, model, num_blocks: int, block_size: int, table_attr: str = "draft_block_table"):
        model.allocate_kv_cache(num_blocks, block_size)
        self.model = model
        self.block_size = block_size
        self.table_attr = table_attr
        self.device = model.device

    def _table(self, seqs) -> torch.Tensor:
        tables = [getattr(s, self.table_attr) for s in seqs]
        width = max(1, max(len(t) for t in tables))
        t = torch.full((len(seqs), width), -1, dtype=torch.int32)
        for b, row in enumerate(tables):
            if row:
                t[b, :len(row)] = torch.as_tensor(row, dtype=torch.int32)
        return t.to(self.device)

    def _slots(self, seqs, pos_rows) -> list[int]:
        bs = self.block_size
        out = []
        for s, p in zip(seqs, pos_rows):
            table = getattr(s, self.table_attr)
            out.append(-1 if p < 0 else table[p // bs] * bs + p % bs)
        return out

    def prefill(self, seqs, chunk: int = 32) -> None:
        """KV of every token but the last of each sequence (the first draft
        step feeds the last one), in chunks of ``chunk`` rows."""
        dev = self.device
        for s in seqs:
            table = self._table([s])
            n = len(s.token_ids) - 1
            for p0 in range(0, n, chunk):
                p1 = min(n, p0 + chunk)
                pos = list(range(p0, p1))
                ids = torch.tensor(s.token_ids[p0:p1], dtype=torch.int64, device=dev)
                self.model.forward(ids, torch.tensor(pos, dtype=torch.int64, device=dev),
                                   torch.tensor(self._slots([s] * len(pos), pos), dtype=torch.int64, device=dev),
                                   table, torch.tensor([p1], dtype=torch.int64, device=dev),
                                   torch.tensor([0, p1 - p0], dtype=torch.int32, device=dev), p1 - p0)

    @torch.inference_mode()
    def run_draft_steps(self, seqs, k: int, temperatures: torch.Tensor,
                        generator: torch.Generator | None = None) -> tuple[list[list[int]], torch.Tensor]:
        """K decode steps for ``seqs`` (n_b confirmed tokens each): step i
        feeds the token at position n_b-1+i and samples draft i+1; step 0
        also re-feeds position n_b-2 (see nsv_prepare_draft).  Returns the
        per-sequence drafts and the logits buffer [k, B, V]."""
        from naivllm_amd.spec_engine.rejection_sampler import sample

        dev, B = self.device, len(seqs)
        table = self._table(seqs)
        V = self.model.cfg.vocab_size
        logit_buf = torch.empty(k, B, V, dtype=self.model.dtype, device=dev)
        tokens = torch.empty(B, k, dtype=torch.int32, device=dev)
        temps = temperatures.to(device=dev, dtype=torch.float32)
        stochastic = bool((temps > 1e-6).any())
        noise = torch.ones(B, V, dtype=torch.float32, device=dev)
        n = [len(s.token_ids) for s in seqs]
        # step 0: rows (n-2, n-1) of every sequence
        pos0 = [p for m in n for p in (m - 2, m - 1)]
        ids0 = [s.token_ids[p] if p >= 0 else 0 for s, m in zip(seqs, n) for p in (m - 2, m - 1)]
        pos0 = [p if p >= 0 else -1 for p in pos0]
        slot0 = self._slots([s for s in seqs for _ in (0, 1)], pos0)
        tmp = self.model.forward(torch.tensor(ids0, dtype=torch.int64, device=dev),
                                 torch.tensor(pos0, dtype=torch.int64, device=dev),
                                 torch.tensor(slot0, dtype=torch.int64, device=dev), table,
                                 torch.tensor(n, dtype=torch.int64, device=dev),
                                 torch.arange(0, 2 * B + 1, 2, dtype=torch.int32, device=dev), 2)
        logit_buf[0].copy_(tmp[1::2])
        cu1 = torch.arange(0, B + 1, dtype=torch.int32, device=dev)
        for i in range(k):
            if i > 0:
                pos = [m - 1 + i for m in n]
                self.model.forward(tokens[:, i - 1], torch.tensor(pos, dtype=torch.int64, device=dev),
                                   torch.tensor(self._slots(seqs, pos), dtype=torch.int64, device=dev), table,
                                   torch.tensor([p + 1 for p in pos], dtype=torch.int64, device=dev), cu1, 1,
                                   logits_out=logit_buf[i])
            if stochastic:
                noise.exponential_(1, generator=generator).clamp_min_(1e-10)
            sample(logit_buf[i], temps, noise, out=tokens[:, i])
        host = tokens.cpu().tolist()  # the one synchronisation of the call
        return host, logit_buf


class ModelDrafter:
    """Draft with a small model running K autoregressive decode steps
    (drafters.py:86-154): same constructor, ``can_draft``, ``prefill`` and
    ``draft`` side effects; ``draft`` returns per-sequence (K, vocab) views
    of the step-major logits buffer, as the reference's fast path."""

    name = "model"

    def __init__(self, runner: DraftRunner, block_manager, num_speculative_tokens: int = 5):
        self.runner = runner
        self.block_manager = block_manager
        self.num_speculative_tokens = num_speculative_tokens
        self.generator: torch.Generator | None = None

    def can_draft(self, seqs, k: int) -> bool:
        return all(self.block_manager.can_ensure_capacity(seq, len(seq) + k + 1) for seq in seqs)

    def prefill(self, seqs) -> None:
        """Mirror the target-side prefill into the draft KV cache."""
        for seq in seqs:
            if not getattr(seq, self.runner.table_attr):
                self.block_manager.allocate(seq)
        for seq in seqs:
            self.block_manager.ensure_capacity(seq, len(seq))
        self.runner.prefill(seqs)

    def draft(self, seqs) -> tuple[list[list[int]], list]:
        k = self.num_speculative_tokens
        if not seqs:
            return [], []
        for seq in seqs:
            self.block_manager.ensure_capacity(seq, len(seq) + k + 1)
        temps = torch.tensor([seq.temperature for seq in seqs], dtype=torch.float32)
        per_seq, logit_buf = self.runner.run_draft_steps(seqs, k, temps, self.generator)
        draft_tokens = []
        for seq, toks in zip(seqs, per_seq):
            seq.draft_tokens = list(toks)
            for t in toks:
                seq.append_token(t)
            draft_tokens.append(list(toks))
        return draft_tokens, [logit_buf[:, j, :] for j in range(len(seqs))]


class HybridDrafter:
    """Cascade drafter (drafters.py:157-196): n-gram lookup first, the model
    drafter for the sequences without a match; ``model_rounds`` /
    ``model_seqs`` count the fallback use."""

    name = "hybrid"

    def __init__(self, ngram: NgramDrafter, model: ModelDrafter):
        self.ngram = ngram
        self.model = model
        self.model_rounds = 0
        self.model_seqs = 0

    def prefill(self, seqs) -> None:
        self.model.prefill(seqs)

    def can_draft(self, seqs, k: int) -> bool:
        return True

    def draft(self, seqs) -> tuple[list[list[int]], list]:
        rows = [None] * len(seqs)
        self.ngram.draft(seqs)
        rest_idx = [i for i, seq in enumerate(seqs) if not seq.draft_tokens]
        if rest_idx:
            rest = [seqs[i] for i in rest_idx]
            if self.model.can_draft(rest, self.model.num_speculative_tokens):
                _, model_rows = self.model.draft(rest)
                self.model_rounds += 1
                self.model_seqs += len(rest)
                for j, i in enumerate(rest_idx):
                    rows[i] = model_rows[j] if j < len(model_rows) else None
        return [list(s.draft_tokens) for s in seqs], rows
