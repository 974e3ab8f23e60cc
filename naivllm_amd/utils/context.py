"""Per-step metadata carrier for the verify forward.

Same fields, defaults and functions as src/myvllm/utils/context.py:6-36:
``set_context`` is how the runner selects the verify kernel and hands it
the row metadata, ``get_context`` is how layers read it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Context:
    is_prefill: bool = False
    is_verify: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    seqlens_q: list[int] | None = None
    seqlens_k: list[int] | None = None
    positions: torch.Tensor | None = None


_context = Context()


def get_context() -> Context:
    return _context


def reset_context() -> None:
    global _context
    _context = Context()


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None, seqlens_q=None, seqlens_k=None,
                is_verify=False, positions=None) -> None:
    global _context
    _context = Context(is_prefill, is_verify, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                       slot_mapping, context_lens, block_tables, seqlens_q, seqlens_k, positions)
