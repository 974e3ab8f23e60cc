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
    spec_llm_engine.py:104-137, model_runner.py:784-847).

    ``run_draft_steps`` is the reference's GPU-resident draft loop
    (``run_draft_steps_gpu``): K decode steps whose sampled tokens feed the
    next step on the device, one host synchronisation per call.  With
    ``use_graphs`` the whole K-step loop (both forwards' kernels and the
    samplers) is captured once per batch bucket {1, 2, 4, ...} and replayed
    from static buffers the host fills each call, as the reference replays
    its decode graph K times from static buffers (model_runner.py:784-847);
    padded rows of a bucket (position -1, slot -1, context 0, table -1) are
    inert.  A call with a caller-supplied generator at a temperature above
    1e-6 runs eagerly, so its draws come from that generator (a captured
    graph draws from torch's device generator)."""

    def __init__(self, model, num_blocks: int, block_size: int, table_attr: str = "draft_block_table",
                 use_graphs: bool = True):
        model.allocate_kv_cache(num_blocks, block_size)
        self.model = model
        self.block_size = block_size
        self.table_attr = table_attr
        self.device = model.device
        self.use_graphs = use_graphs
        self._bufs: dict | None = None
        self._graphs: dict = {}  # (bucket, stochastic) -> captured graph

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

    def prefill(self, seqs, starts=None) -> None:
        """KV of the tokens of each sequence from ``starts[i]`` (default 0: the
        draft pool's own prefix is empty) in one forward over every sequence
        (Qwen3Verify.prefill: causal blocks through the verify kernel)."""
        if not seqs:
            return
        starts = [0] * len(seqs) if starts is None else list(starts)
        self.model.prefill([s.token_ids for s in seqs], starts, [getattr(s, self.table_attr) for s in seqs])

    # ----------------------------------------------------------- draft loop
    def _ensure_bufs(self, B: int, k: int, width: int) -> dict:
        b = self._bufs
        if b is not None and b["max_batch"] >= B and b["k"] == k and b["width"] >= width:
            return b
        mb = 1
        while mb < B:
            mb *= 2
        if b is not None:
            mb = max(mb, b["max_batch"])
            width = max(width, b["width"])
        dev, V = self.device, self.model.cfg.vocab_size
        i64 = dict(dtype=torch.int64, device=dev)
        b = {"max_batch": mb, "k": k, "width": width,
             "ids0": torch.zeros(2 * mb, **i64), "pos0": torch.full((2 * mb,), -1, **i64),
             "slot0": torch.full((2 * mb,), -1, **i64), "ctx0": torch.zeros(mb, **i64),
             "pos": torch.full((k, mb), -1, **i64), "slot": torch.full((k, mb), -1, **i64),
             "ctx": torch.zeros(k, mb, **i64),
             "table": torch.full((mb, width), -1, dtype=torch.int32, device=dev),
             "temps": torch.zeros(mb, dtype=torch.float32, device=dev),
             "noise": torch.ones(mb, V, dtype=torch.float32, device=dev),
             "tokens": torch.zeros(mb, k, dtype=torch.int32, device=dev),
             "logits": torch.empty(k, mb, V, dtype=self.model.dtype, device=dev),
             "cu2": torch.arange(0, 2 * mb + 1, 2, dtype=torch.int32, device=dev),
             "cu1": torch.arange(0, mb + 1, dtype=torch.int32, device=dev)}
        self._bufs = b
        self._graphs = {}  # captured over the previous buffers
        return b

    def _body(self, b: dict, Bb: int, stochastic: bool, generator=None) -> None:
        """The K steps over the first Bb rows of the static buffers: step 0
        feeds positions (n-2, n-1) of every sequence, step i > 0 the token
        step i - 1 sampled."""
        from naivllm_amd.spec_engine.rejection_sampler import sample

        k, m = b["k"], self.model
        noise = b["noise"][:Bb]
        tmp = m.forward(b["ids0"][:2 * Bb], b["pos0"][:2 * Bb], b["slot0"][:2 * Bb], b["table"][:Bb], b["ctx0"][:Bb],
                        b["cu2"][:Bb + 1], 2)
        b["logits"][0, :Bb].copy_(tmp[1::2])
        for i in range(k):
            if i > 0:
                m.forward(b["tokens"][:Bb, i - 1], b["pos"][i, :Bb], b["slot"][i, :Bb], b["table"][:Bb],
                          b["ctx"][i, :Bb], b["cu1"][:Bb + 1], 1, logits_out=b["logits"][i, :Bb])
            if stochastic:
                noise.exponential_(1, generator=generator).clamp_min_(1e-10)
            sample(b["logits"][i, :Bb], b["temps"][:Bb], noise, out=b["tokens"][:Bb, i])

    @torch.inference_mode()
    def run_draft_steps(self, seqs, k: int, temperatures: torch.Tensor,
                        generator: torch.Generator | None = None) -> tuple[list[list[int]], torch.Tensor]:
        """K decode steps for ``seqs`` (n_b confirmed tokens each): step i
        feeds the token at position n_b-1+i and samples draft i+1; step 0
        also re-feeds position n_b-2 (see nsv_prepare_draft).  Returns the
        per-sequence drafts and the logits buffer [k, B, V] (valid until the
        next call)."""
        import numpy as np

        B = len(seqs)
        temps = temperatures.to(dtype=torch.float32).cpu()
        stochastic = bool((temps > 1e-6).any())
        tables = [getattr(s, self.table_attr) for s in seqs]
        width = max(1, max(len(t) for t in tables))
        b = self._ensure_bufs(B, k, width)
        Bb = 1
        while Bb < B:
            Bb *= 2
        # host staging of the call's metadata (pad rows inert)
        n = np.array([len(s.token_ids) for s in seqs], dtype=np.int64)
        p0 = np.stack([n - 2, n - 1], axis=1).reshape(-1)
        ids0 = np.zeros(2 * Bb, dtype=np.int64)
        pos0 = np.full(2 * Bb, -1, dtype=np.int64)
        slot0 = np.full(2 * Bb, -1, dtype=np.int64)
        for j, s in enumerate(seqs):
            for r in (0, 1):
                p = int(p0[2 * j + r])
                if p >= 0:
                    ids0[2 * j + r] = s.token_ids[p]
                    pos0[2 * j + r] = p
        slot0[:2 * B] = self._slots([s for s in seqs for _ in (0, 1)], pos0[:2 * B].tolist())
        pos = np.full((k, Bb), -1, dtype=np.int64)
        slot = np.full((k, Bb), -1, dtype=np.int64)
        ctx = np.zeros((k, Bb), dtype=np.int64)
        for i in range(1, k):
            pi = (n - 1 + i).tolist()
            pos[i, :B] = pi
            slot[i, :B] = self._slots(seqs, pi)
            ctx[i, :B] = n + i
        ctx0 = np.zeros(Bb, dtype=np.int64)
        ctx0[:B] = n
        table = np.full((Bb, b["width"]), -1, dtype=np.int32)
        for j, row in enumerate(tables):
            table[j, :len(row)] = row
        tv = np.zeros(Bb, dtype=np.float32)
        tv[:B] = temps.numpy()
        dev = self.device
        t = lambda x: torch.from_numpy(x).to(dev, non_blocking=False)  # noqa: E731
        b["ids0"][:2 * Bb].copy_(t(ids0))
        b["pos0"][:2 * Bb].copy_(t(pos0))
        b["slot0"][:2 * Bb].copy_(t(slot0))
        b["ctx0"][:Bb].copy_(t(ctx0))
        b["pos"][:, :Bb].copy_(t(pos))
        b["slot"][:, :Bb].copy_(t(slot))
        b["ctx"][:, :Bb].copy_(t(ctx))
        b["table"][:Bb].copy_(t(table))
        b["temps"][:Bb].copy_(t(tv))
        if not stochastic:
            b["noise"][:Bb].fill_(1.0)
        if not self.use_graphs or (stochastic and generator is not None):
            self._body(b, Bb, stochastic, generator)
        else:
            key = (Bb, stochastic)
            graph = self._graphs.get(key)
            if graph is None:
                self._body(b, Bb, stochastic)  # warm-up (workspaces sized); its results stand for this call
                torch.cuda.synchronize(dev)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    self._body(b, Bb, stochastic)
                self._graphs[key] = graph
                # the capture did not run; this call's results are the warm-up's
            else:
                graph.replay()
        host = b["tokens"][:B].cpu().tolist()  # the one synchronisation of the call
        return host, b["logits"][:, :B]


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
