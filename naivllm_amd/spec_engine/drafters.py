"""Token drafters on the GPU.

``NgramDrafter`` keeps the reference's interface and side effects
(src/myvllm/spec_engine/drafters.py:26-61): ``draft(seqs)`` appends each
sequence's drafts with ``append_token``, records them in
``seq.draft_tokens`` and returns ``(drafts, [None] * len(seqs))``.  The
lookup itself (the reference's ``_lookup``, :63-83, a ``bytes.rfind`` over
the big-endian uint32 encoding of the history) runs as one GPU kernel over
the whole batch; ``draft_device`` is the device-resident form the
verification round uses on a history that never leaves the GPU.
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
