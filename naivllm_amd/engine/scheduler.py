"""Request scheduler: waiting / running queues over a BlockManager.

Drop-in for src/myvllm/engine/scheduler.py (:6-98), same constructor,
queues and methods:
  * ``schedule()`` admits waiting sequences for prefill while they fit
    ``max_num_sequences`` and ``max_num_batched_tokens`` (counting only the
    prompt tokens the prefix cache does not serve) and their pages can be
    allocated; with none admitted it schedules running sequences for one
    decode token each, preempting the lowest-priority running sequence
    (the last in the queue) when a page cannot be appended;
  * ``preempt(seq)`` frees its pages and puts it back at the front of the
    waiting queue;
  * ``postprocess(seqs, token_ids)`` appends each sequence's new token and
    finishes it on EOS (unless ignore_eos), max_tokens or max_model_length.

The speculative engine (naivllm_amd.spec_engine.SpecLLMEngine) uses the
same queues: admission goes through ``admit()`` (the prefill half of
``schedule()``, with each admitted sequence's whole speculative page
reservation checked as well), and decoding is the device-resident round.
"""

from __future__ import annotations

from collections import deque

from naivllm_amd.engine.block_manager import BlockManager
from naivllm_amd.engine.sequence import Sequence, SequenceStatus


class Scheduler:
    def __init__(self, max_num_sequences: int, max_num_batched_tokens: int, max_cached_blocks: int, block_size: int,
                 eos: int):
        self.block_manager = BlockManager(max_cached_blocks, block_size)
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_num_sequences = max_num_sequences
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        self.eos = eos

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def add_sequence(self, sequence: Sequence) -> None:
        self.waiting.append(sequence)

    def admit(self, max_new: int, reserve=None) -> list[Sequence]:
        """Admit waiting sequences, in order, for prefill: at most ``max_new``
        of them, within the token budget (uncached prompt tokens) and the
        free pages; ``reserve(seq)`` (optional) returns the number of tokens
        the sequence's pages must cover once admitted, checked against the
        pages left after its allocation."""
        admitted: list[Sequence] = []
        budget = 0
        bm = self.block_manager
        while self.waiting and len(admitted) < max_new:
            seq = self.waiting[0]
            if not bm.can_allocate(seq):
                break
            new_tokens = len(seq) - len(bm._cached_prefix(seq)) * bm.block_size
            if admitted and budget + new_tokens > self.max_num_batched_tokens:
                break
            bm.allocate(seq)
            if reserve is not None and not bm.can_ensure_capacity(seq, reserve(seq)):
                bm.deallocate(seq)
                break
            if reserve is not None:
                bm.ensure_capacity(seq, reserve(seq))
            self.waiting.popleft()
            seq.status = SequenceStatus.RUNNING
            self.running.append(seq)
            admitted.append(seq)
            budget += new_tokens
        return admitted

    def schedule(self) -> tuple[list[Sequence], bool]:
        scheduled: list[Sequence] = []
        tokens = 0
        bm = self.block_manager
        while self.waiting and len(scheduled) < self.max_num_sequences:
            seq = self.waiting[0]
            if not bm.can_allocate(seq):
                break
            new_tokens = len(seq) - len(bm._cached_prefix(seq)) * bm.block_size
            if new_tokens + tokens > self.max_num_batched_tokens:
                break
            self.waiting.popleft()
            bm.allocate(seq)
            seq.status = SequenceStatus.RUNNING
            self.running.append(seq)
            scheduled.append(seq)
            tokens += new_tokens
        if scheduled:
            return scheduled, True

        while self.running and tokens < self.max_num_batched_tokens and len(scheduled) < self.max_num_sequences:
            seq = self.running[0]
            if not bm.can_append(seq):
                victim = self.running.pop()  # the lowest priority: last in the queue
                self.preempt(victim)
                if victim is seq:
                    break
                continue
            bm.append(seq)
            scheduled.append(seq)
            tokens += 1
            self.running.popleft()
        if scheduled:
            self.running.extendleft(reversed(scheduled))
        return scheduled, False

    def preempt(self, seq: Sequence) -> None:
        self.block_manager.deallocate(seq)
        seq.status = SequenceStatus.WAITING
        self.waiting.appendleft(seq)

    def finish(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.FINISHED
        self.block_manager.deallocate(seq)
        if seq in self.running:
            self.running.remove(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int]) -> None:
        for seq, token_id in zip(seqs, token_ids):
            seq.append_token(token_id)
            stop_eos = not seq.ignore_eos and token_id == self.eos
            stop_max_tokens = seq.num_completion_tokens >= seq.max_tokens
            stop_max_length = seq.max_model_length is not None and seq.num_tokens >= seq.max_model_length
            if stop_eos or stop_max_tokens or stop_max_length:
                self.finish(seq)
