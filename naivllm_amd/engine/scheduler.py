"""Request queues over a BlockManager: admission, decode steps, preemption.

Interface of src/myvllm/engine/scheduler.py (:6-98): the constructor
arguments, the ``waiting`` / ``running`` deques, ``add_sequence``,
``is_finished``, ``schedule() -> (sequences, is_prefill)``, ``preempt`` and
``postprocess`` keep the reference's names and meaning, so its engine loop
(engine/llm_engine.py:64-75) drives this class unchanged.  The policy:

* **Admission** (``admit``; the prefill half of ``schedule``).  Requests are
  taken from the head of the waiting queue, in order, and admission stops at
  the first that does not fit.  A request fits when the batch stays within
  the caller's slot count, the token budget (``max_num_batched_tokens``,
  counted in prompt tokens the prefix cache does not serve; the first
  request of a batch is always within budget, so a prompt longer than the
  budget is not starved) and the free pages.  Pages are counted for the
  whole reservation before anything is allocated: the prompt, or the
  caller's ``reserve(seq)`` token count when that is larger, less the
  prefix-cache hits, plus the cached hits that sit in the free queue (taking
  one removes a free page).  A request that does not fit changes nothing.
* **Decode step** (``schedule`` when nothing was admitted).  The step is the
  first ``min(max_num_sequences, max_num_batched_tokens)`` running
  sequences (one token each).  Its page demand is the number of pages its
  sequences' tables lack for their token counts.  While the demand exceeds
  the free pages, the lowest-priority running sequence (the back of the
  queue) is preempted, which frees its pages and, when it was part of the
  step, shrinks the step.  Then every sequence of the step gets its page.
  The running queue keeps its order.
* **Preemption** returns a sequence's pages and puts it at the head of the
  waiting queue, so it is the next to be prefilled again.
* **Completion** (``postprocess``) appends each sampled token and finishes
  the sequence on EOS (unless ``ignore_eos``), on ``max_tokens`` completion
  tokens, or on reaching ``max_model_length`` tokens; a finished sequence
  returns its pages.

The speculative engine (naivllm_amd.spec_engine.SpecLLMEngine) admits through
``admit()`` with each request's whole speculative reservation and decodes in
the device-resident round, so it calls ``finish`` itself.
"""

from __future__ import annotations

from collections import deque
from itertools import islice

from naivllm_amd.engine.block_manager import BlockManager
from naivllm_amd.engine.sequence import Sequence, SequenceStatus


class Scheduler:
    def __init__(self, max_num_sequences: int, max_num_batched_tokens: int, max_cached_blocks: int, block_size: int,
                 eos: int):
        self.max_num_sequences = max_num_sequences
        self.max_num_batched_tokens = max_num_batched_tokens
        self.eos = eos
        self.block_manager = BlockManager(max_cached_blocks, block_size)
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()

    # ------------------------------------------------------------------ queues
    def is_finished(self) -> bool:
        return len(self.waiting) + len(self.running) == 0

    def add_sequence(self, sequence: Sequence) -> None:
        self.waiting.append(sequence)

    # --------------------------------------------------------------- admission
    def admit(self, max_new: int, reserve=None) -> list[Sequence]:
        """Admit up to ``max_new`` waiting requests for prefill (policy in the
        module docstring).  ``reserve(seq)``, if given, is the number of token
        positions the request's pages must cover from admission on."""
        bm = self.block_manager
        batch: list[Sequence] = []
        spent = 0
        while self.waiting and len(batch) < max_new:
            head = self.waiting[0]
            cover = len(head) if reserve is None else max(len(head), reserve(head))
            if not bm.can_allocate(head, cover):
                break
            uncached = bm.uncached_tokens(head)
            if batch and spent + uncached > self.max_num_batched_tokens:
                break
            bm.allocate(head)
            bm.ensure_capacity(head, cover)
            self.waiting.popleft()
            head.status = SequenceStatus.RUNNING
            self.running.append(head)
            batch.append(head)
            spent += uncached
        return batch

    def _decode_step(self) -> list[Sequence]:
        """The running sequences that take one token this step, each given the
        page its newest token needs (policy in the module docstring)."""
        bm = self.block_manager
        width = min(self.max_num_sequences, self.max_num_batched_tokens)
        step: list[Sequence] = []
        while self.running:
            step = list(islice(self.running, width))
            demand = sum(bm.pages_short(s) for s in step)
            if demand <= len(bm.free_block_ids):
                break
            self.preempt(self.running[-1])
            step = []
        for s in step:
            bm.append(s)
        return step

    def schedule(self) -> tuple[list[Sequence], bool]:
        """Prefill the requests that can be admitted, else one decode step:
        ``(sequences, is_prefill)``."""
        admitted = self.admit(self.max_num_sequences)
        if admitted:
            return admitted, True
        return self._decode_step(), False

    # -------------------------------------------------------- leaving the queue
    def preempt(self, seq: Sequence) -> None:
        """Return the sequence's pages and requeue it at the head of the waiting
        queue (its prompt and output so far are prefilled again)."""
        if seq in self.running:
            self.running.remove(seq)
        self.block_manager.deallocate(seq)
        seq.status = SequenceStatus.WAITING
        self.waiting.appendleft(seq)

    def finish(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.FINISHED
        self.block_manager.deallocate(seq)
        if seq in self.running:
            self.running.remove(seq)

    def _stops(self, seq: Sequence, token_id: int) -> bool:
        if token_id == self.eos and not seq.ignore_eos:
            return True
        if seq.num_completion_tokens >= seq.max_tokens:
            return True
        return seq.max_model_length is not None and seq.num_tokens >= seq.max_model_length

    def postprocess(self, seqs: list[Sequence], token_ids: list[int]) -> None:
        """Append each sequence's sampled token; finish the ones that stop."""
        for seq, token_id in zip(seqs, token_ids):
            seq.append_token(token_id)
            if self._stops(seq, token_id):
                self.finish(seq)
