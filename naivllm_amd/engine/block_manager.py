"""Paged-KV page bookkeeping on the host.

Same behaviour as the parts of src/myvllm/engine/block_manager.py the
verification round uses: ``allocate`` (pages for a new sequence),
``deallocate``, ``append`` (a page for the next token), and the speculative
capacity API ``can_ensure_capacity`` / ``ensure_capacity`` (:245-257),
``rollback`` (:259-269) and ``trim_to`` (:273-300).  The reference's
xxhash prefix cache and prefix pinning (:120-188) are not part of the round
and are not built: pages here are never shared, so every page has one owner.
``table_attr`` selects the Sequence attribute holding the page list, so a
draft model can keep its own table (``draft_block_table``).
"""

from __future__ import annotations

from collections import deque


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int, table_attr: str = "block_table",
                 cached_attr: str = "num_cached_tokens"):
        self.block_size = block_size
        self.table_attr = table_attr
        self.cached_attr = cached_attr
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()

    def _table(self, seq) -> list[int]:
        return getattr(seq, self.table_attr)

    def _take(self) -> int:
        block_id = self.free_block_ids.popleft()
        self.used_block_ids.add(block_id)
        return block_id

    def _release(self, block_id: int) -> None:
        self.used_block_ids.discard(block_id)
        self.free_block_ids.append(block_id)

    def _pages_for(self, num_tokens: int) -> int:
        return (num_tokens + self.block_size - 1) // self.block_size

    def can_allocate(self, seq) -> bool:
        return len(self.free_block_ids) >= self._pages_for(len(seq))

    def allocate(self, seq) -> None:
        assert not self._table(seq), "sequence already has pages"
        for _ in range(self._pages_for(len(seq))):
            self._table(seq).append(self._take())
        setattr(seq, self.cached_attr, 0)

    def deallocate(self, seq) -> None:
        table = self._table(seq)
        while table:
            self._release(table.pop())
        setattr(seq, self.cached_attr, 0)

    def can_append(self, seq) -> bool:
        return len(self.free_block_ids) >= (1 if len(self._table(seq)) < seq.num_blocks else 0)

    def append(self, seq) -> None:
        """Give the sequence a page for its newest token if it crossed into
        one it does not have yet."""
        if len(self._table(seq)) < seq.num_blocks:
            self._table(seq).append(self._take())

    def _blocks_needed_for(self, seq, target_num_tokens: int) -> int:
        return max(0, self._pages_for(target_num_tokens) - len(self._table(seq)))

    def can_ensure_capacity(self, seq, target_num_tokens: int) -> bool:
        return len(self.free_block_ids) >= self._blocks_needed_for(seq, target_num_tokens)

    def ensure_capacity(self, seq, target_num_tokens: int) -> None:
        """Extend the table to cover ``target_num_tokens`` positions (before a
        multi-token verify forward)."""
        for _ in range(self._blocks_needed_for(seq, target_num_tokens)):
            self._table(seq).append(self._take())

    def rollback(self, seq, num_tokens: int) -> None:
        """Drop the last ``num_tokens`` completion tokens and the pages no
        longer needed."""
        if num_tokens <= 0:
            return
        if num_tokens > seq.num_completion_tokens:
            raise ValueError("rollback cannot remove prompt tokens")
        seq.token_ids = seq.token_ids[:-num_tokens]
        seq.num_tokens -= num_tokens
        seq.last_token = seq.token_ids[-1]
        self.trim_to(seq, seq.num_tokens)

    def trim_to(self, seq, new_num_tokens: int) -> None:
        """Release pages beyond what ``new_num_tokens`` needs (token_ids is
        the caller's)."""
        table = self._table(seq)
        while len(table) > self._pages_for(new_num_tokens):
            self._release(table.pop())
