"""Paged-KV page bookkeeping on the host, with prefix caching.

Drop-in for src/myvllm/engine/block_manager.py (same class, method names,
arguments and observable state, since the reference's callers and tests
read them: ``blocks[i].token_ids``, ``free_block_ids``, ``used_block_ids``,
``cache_stats()``, ``seq.block_table``, ``seq.num_cached_tokens``):

  * prefix cache (:58-160): a full page is keyed by the xxh64 hash of its
    int32 token ids chained onto the previous page's hash; a new sequence
    reuses every leading full page whose hash and tokens match, except
    that the page holding its last token is always recomputed (the model
    must see at least one token to produce the next);
  * pinning (:169-197): ``pin_prefix`` keeps the cached full pages of a
    token prefix resident (out of the free pool) until ``unpin_all``;
  * speculative capacity (:245-257), ``rollback`` (:259-269) and
    ``trim_to`` (:273-300), which clears the hash of a partial tail page and
    finalises it when the confirmed tokens end exactly on a page boundary;
  * ``append`` (:207-237) finalises a page's hash when it fills.

Freed pages keep their hash and tokens and go to the back of the free
queue, so a later request can still find them until they are reused.
Two deliberate differences: prefix reuse stops at the first page that
misses (the reference keeps looking and can count a later page as cached
after a miss, which would make num_cached_tokens cover pages that are not
a prefix), and ``can_append`` asks for a page exactly when the newest token
needs one (see there).

``register_full_pages`` is this build's addition for the device-resident
round, whose tokens land on the host only when a sequence finishes: it
hashes every page of the final token list whose KV is complete (the
reference hashes them one by one in ``append`` as decoding fills them).
``can_allocate`` takes an optional reservation and counts the cached hits
that must be taken out of the free queue; ``free_pages_needed``,
``uncached_tokens`` and ``pages_short`` are the scheduler's page arithmetic.
"""

from __future__ import annotations

from collections import deque

import numpy as np
import xxhash


class Block:
    """One KV page: id, prefix hash (-1 = none), references, pins, tokens."""

    __slots__ = ("block_id", "hash", "ref_count", "pin_count", "token_ids")

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.hash = -1
        self.ref_count = 0
        self.pin_count = 0
        self.token_ids: list[int] = []

    def update(self, h: int, token_ids: list[int]) -> None:
        self.hash = h
        self.token_ids = token_ids

    def reset(self) -> None:
        self.hash = -1
        self.ref_count = 0
        self.pin_count = 0
        self.token_ids = []


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int, table_attr: str = "block_table",
                 cached_attr: str = "num_cached_tokens"):
        self.block_size = block_size
        self.table_attr = table_attr
        self.cached_attr = cached_attr
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()
        self.cache_hits = 0
        self.cache_misses = 0

    # ----------------------------------------------------------------- helpers
    def _table(self, seq) -> list[int]:
        return getattr(seq, self.table_attr)

    def _cached(self, seq) -> int:
        return getattr(seq, self.cached_attr)

    def _pages_for(self, num_tokens: int) -> int:
        return (num_tokens + self.block_size - 1) // self.block_size

    def compute_hash(self, token_ids: list[int], prefix_hash_value: int = -1) -> int:
        h = xxhash.xxh64()
        if prefix_hash_value != -1:
            h.update(int(prefix_hash_value).to_bytes(8, "little"))
        h.update(np.asarray(token_ids, dtype=np.int32).tobytes())
        return h.intdigest()

    def _take_fresh(self) -> Block:
        """The page at the front of the free queue, cleared, with one reference."""
        block_id = self.free_block_ids[0]
        block = self.blocks[block_id]
        assert block.ref_count == 0, "Block is already allocated"
        block.reset()
        self.free_block_ids.popleft()
        self.used_block_ids.add(block_id)
        block.ref_count = 1
        return block

    def _acquire_cached(self, block_id: int) -> Block:
        """One more reference to a page, keeping its hash and tokens."""
        block = self.blocks[block_id]
        if block_id not in self.used_block_ids:
            self.free_block_ids.remove(block_id)
            self.used_block_ids.add(block_id)
        block.ref_count += 1
        return block

    def _release(self, block_id: int) -> None:
        block = self.blocks[block_id]
        block.ref_count -= 1
        if block.ref_count == 0:
            self.used_block_ids.discard(block_id)
            self.free_block_ids.append(block_id)

    def _cached_prefix(self, seq) -> list[int]:
        """Ids of the cached pages the sequence may reuse: its leading full
        pages found in the cache with equal tokens, none covering its last
        token."""
        out = []
        h = -1
        limit = seq.num_tokens - 1  # at least the last token is recomputed
        for i in range(seq.num_blocks):
            tokens = seq.block(i)
            if len(tokens) != self.block_size or (i + 1) * self.block_size > limit:
                break
            h = self.compute_hash(tokens, h)
            block_id = self.hash_to_block_id.get(h, -1)
            if block_id == -1 or self.blocks[block_id].token_ids != tokens:
                break
            out.append(block_id)
        return out

    # -------------------------------------------------------------- allocation
    def free_pages_needed(self, seq, num_tokens: int = 0) -> int:
        """Free pages that allocating ``seq`` with room for
        ``max(num_tokens, len(seq))`` positions takes out of the free queue:
        the pages the prefix cache does not serve, plus every cached hit no
        sequence holds (it sits in the free queue until taken)."""
        seq.block_size = self.block_size
        hits = self._cached_prefix(seq)
        pages = self._pages_for(max(num_tokens, seq.num_tokens))
        idle_hits = sum(1 for b in hits if self.blocks[b].ref_count == 0)
        return pages - len(hits) + idle_hits

    def can_allocate(self, seq, num_tokens: int = 0) -> bool:
        """Whether ``allocate`` (then ``ensure_capacity(seq, num_tokens)``)
        finds enough free pages.  (The reference compares the free pages with
        the missing pages only, so a hit taken from the free queue can leave
        ``allocate`` short.)"""
        return len(self.free_block_ids) >= self.free_pages_needed(seq, num_tokens)

    def uncached_tokens(self, seq) -> int:
        """Prompt tokens the prefix cache does not serve (the prefill's work)."""
        seq.block_size = self.block_size
        return seq.num_tokens - len(self._cached_prefix(seq)) * self.block_size

    def allocate(self, seq) -> None:
        seq.block_size = self.block_size
        table = self._table(seq)
        assert not table, "sequence already has pages"
        hits = self._cached_prefix(seq)
        for block_id in hits:
            self._acquire_cached(block_id)
            table.append(block_id)
            self.cache_hits += 1
        setattr(seq, self.cached_attr, len(hits) * self.block_size)
        h = self.blocks[hits[-1]].hash if hits else -1
        for i in range(len(hits), seq.num_blocks):
            tokens = seq.block(i)
            block = self._take_fresh()
            self.cache_misses += 1
            if len(tokens) == self.block_size:
                h = self.compute_hash(tokens, h)
                block.update(h, tokens)
                self.hash_to_block_id[h] = block.block_id
            else:
                h = -1
            table.append(block.block_id)

    def deallocate(self, seq) -> None:
        for block_id in self._table(seq):  # table order, as the reference releases them
            self._release(block_id)
        setattr(seq, self.table_attr, [])
        setattr(seq, self.cached_attr, 0)

    # ------------------------------------------------------------------ pinning
    def pin_prefix(self, token_ids: list[int]) -> int:
        """Pin the cached full pages of ``token_ids`` (leading, matching) so
        they are never returned to the free pool; returns the tokens they
        cover.  The prefix must have been evaluated before (its pages exist)."""
        h = -1
        pinned = 0
        for start in range(0, len(token_ids) - self.block_size + 1, self.block_size):
            tokens = list(token_ids[start:start + self.block_size])
            h = self.compute_hash(tokens, h)
            block_id = self.hash_to_block_id.get(h, -1)
            if block_id == -1 or self.blocks[block_id].token_ids != tokens:
                break
            block = self.blocks[block_id]
            if block.pin_count == 0:
                self._acquire_cached(block_id)
            block.pin_count += 1
            pinned += self.block_size
        return pinned

    def unpin_all(self) -> None:
        for block in self.blocks:
            if block.pin_count:
                block.pin_count = 0
                self._release(block.block_id)

    def cache_stats(self) -> dict[str, int]:
        return {
            "hits": self.cache_hits,
            "misses": self.cache_misses,
            "pinned_blocks": sum(1 for b in self.blocks if b.pin_count > 0),
            "free_blocks": len(self.free_block_ids),
        }

    # ------------------------------------------------------------ token growth
    def pages_short(self, seq) -> int:
        """Pages the sequence's table lacks for its token count."""
        return max(0, seq.num_blocks - len(self._table(seq)))

    def can_append(self, seq) -> bool:
        """Whether ``append`` can give the newest token its page: a free page
        is needed exactly when the token crossed into a page the table does
        not have yet.  (The reference tests num_tokens % block_size == 0,
        one token early: it asks for a page when none is needed and answers
        True when one is, after which append runs out of pages.)"""
        if len(self._table(seq)) < seq.num_blocks:
            return len(self.free_block_ids) > 0
        return True

    def _finalize_last(self, seq, num_pages: int) -> None:
        """Hash page num_pages - 1 of the table, now full, chained onto the
        page before it, and register it in the cache."""
        table = self._table(seq)
        block = self.blocks[table[num_pages - 1]]
        prev = self.blocks[table[num_pages - 2]].hash if num_pages > 1 else -1
        tokens = seq.block(num_pages - 1)
        h = self.compute_hash(tokens, prev)
        block.update(h, tokens)
        self.hash_to_block_id[h] = block.block_id

    def append(self, seq) -> None:
        """After a token was appended to the sequence: finalise the page it
        filled, or give it a page for a token that crossed into a new one."""
        table = self._table(seq)
        n = seq.num_tokens
        if n % self.block_size == 0:
            if self.blocks[table[-1]].hash == -1:
                self._finalize_last(seq, len(table))
        elif len(table) < seq.num_blocks:
            table.append(self._take_fresh().block_id)
        else:
            assert table[-1] in self.used_block_ids, "Last block should be allocated"
            assert self.blocks[table[-1]].hash == -1, "Last block should be partial block with hash -1"

    def register_full_pages(self, seq) -> None:
        """Hash, in order, every page of the sequence that has no hash yet and
        whose tokens all have their KV written, so later requests can reuse
        it.  The device round writes a token's KV in the round after the one
        that committed it (its verify rows are [last confirmed, drafts]), so
        the last token never has KV of its own: a page is registered only when
        it ends before the last token."""
        table = self._table(seq)
        full = min(max(seq.num_tokens - 1, 0) // self.block_size, len(table))
        for i in range(full):
            if self.blocks[table[i]].hash == -1:
                self._finalize_last(seq, i + 1)

    # ---------------------------------------------------- speculative capacity
    def _blocks_needed_for(self, seq, target_num_tokens: int) -> int:
        return max(0, self._pages_for(target_num_tokens) - len(self._table(seq)))

    def can_ensure_capacity(self, seq, target_num_tokens: int) -> bool:
        return len(self.free_block_ids) >= self._blocks_needed_for(seq, target_num_tokens)

    def ensure_capacity(self, seq, target_num_tokens: int) -> None:
        """Extend the table to cover ``target_num_tokens`` positions (before a
        multi-token verify forward); new pages carry no hash."""
        for _ in range(self._blocks_needed_for(seq, target_num_tokens)):
            self._table(seq).append(self._take_fresh().block_id)

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
        the caller's); a partial tail page loses its hash, a tail page the
        confirmed tokens fill exactly is hashed."""
        needed = self._pages_for(new_num_tokens)
        table = self._table(seq)
        while len(table) > needed:
            self._release(table.pop())
        if not table:
            return
        if new_num_tokens % self.block_size:
            block = self.blocks[table[-1]]
            if block.hash != -1 and self.hash_to_block_id.get(block.hash) == block.block_id:
                del self.hash_to_block_id[block.hash]
            block.hash = -1
            block.token_ids = []
        else:
            self._finalize_last(seq, needed)
