"""Host bookkeeping of pages and requests on the CPU: the reference's own
block-manager and scheduler tests (tests/test_block_manager.py:5-53,
tests/test_scheduler.py:6-17 of the reference), restated against
naivllm_amd, plus the prefix-cache, pinning and speculative-capacity
semantics of src/myvllm/engine/block_manager.py."""

import pytest

from naivllm_amd.engine.block_manager import BlockManager
from naivllm_amd.engine.scheduler import Scheduler
from naivllm_amd.engine.sequence import Sequence
from naivllm_amd.sampling_parameters import SamplingParams


# ---- the reference's tests ---------------------------------------------------
def test_exact_multiple_has_a_full_last_block():
    sequence = Sequence([1, 2, 3, 4])
    sequence.block_size = 4
    assert sequence.last_block_num_tokens == 4
    assert sequence.block(0) == [1, 2, 3, 4]


def test_cached_block_survives_release_and_is_reused():
    manager = BlockManager(num_blocks=4, block_size=4)
    first = Sequence([1, 2, 3, 4, 5])
    manager.allocate(first)
    cached_id = first.block_table[0]
    manager.deallocate(first)

    second = Sequence([1, 2, 3, 4, 9])
    manager.allocate(second)

    assert second.block_table[0] == cached_id
    assert second.num_cached_tokens == 4
    assert manager.blocks[cached_id].token_ids == [1, 2, 3, 4]
    assert manager.cache_stats()["hits"] == 1


def test_pinned_prefix_is_not_returned_to_free_pool():
    manager = BlockManager(num_blocks=4, block_size=4)
    sequence = Sequence([1, 2, 3, 4, 5])
    manager.allocate(sequence)
    prefix_id = sequence.block_table[0]
    manager.deallocate(sequence)

    assert manager.pin_prefix([1, 2, 3, 4]) == 4
    assert prefix_id in manager.used_block_ids
    assert prefix_id not in manager.free_block_ids

    manager.unpin_all()
    assert prefix_id in manager.free_block_ids


def test_rollback_releases_extra_blocks():
    manager = BlockManager(num_blocks=4, block_size=4)
    sequence = Sequence([1, 2, 3, 4])
    manager.allocate(sequence)
    sequence.append_token(5)
    manager.append(sequence)

    manager.rollback(sequence, 1)

    assert sequence.token_ids == [1, 2, 3, 4]
    assert len(sequence.block_table) == 1


def test_max_tokens_is_not_off_by_one():
    scheduler = Scheduler(1, 32, 8, 4, eos=99)
    sequence = Sequence([1, 2], SamplingParams(max_tokens=2, ignore_eos=True))
    scheduler.add_sequence(sequence)
    scheduled, _ = scheduler.schedule()
    scheduler.postprocess(scheduled, [3])
    assert not sequence.is_finished

    scheduled, _ = scheduler.schedule()
    scheduler.postprocess(scheduled, [4])
    assert sequence.is_finished
    assert sequence.completion_token_ids == [3, 4]


# ---- prefix cache semantics --------------------------------------------------
def test_last_token_is_never_served_from_cache():
    # a prompt of exactly two full pages reuses only the first: the page
    # holding its last token is recomputed so the model sees one token
    m = BlockManager(8, 4)
    a = Sequence(list(range(8)))
    m.allocate(a)
    first_page = a.block_table[0]
    m.deallocate(a)
    b = Sequence(list(range(8)))
    m.allocate(b)
    assert b.num_cached_tokens == 4 and b.block_table[0] == first_page
    assert m.cache_stats()["hits"] == 1 and m.cache_stats()["misses"] == 3


def test_hashes_chain_on_the_prefix():
    # the same page content after a different first page is a different page
    m = BlockManager(8, 4)
    a = Sequence([1, 2, 3, 4, 5, 6, 7, 8, 9])
    m.allocate(a)
    b = Sequence([0, 0, 0, 0, 5, 6, 7, 8, 9])
    m.allocate(b)
    assert b.num_cached_tokens == 0
    assert set(a.block_table).isdisjoint(b.block_table)
    c = Sequence([1, 2, 3, 4, 5, 6, 7, 8, 1, 2])
    m.allocate(c)  # shares both full pages of a while a still runs
    assert c.block_table[:2] == a.block_table[:2] and c.num_cached_tokens == 8
    assert m.blocks[a.block_table[0]].ref_count == 2


def test_reuse_stops_at_the_first_miss():
    m = BlockManager(8, 4)
    a = Sequence([1, 2, 3, 4, 5, 6, 7, 8, 9])
    m.allocate(a)
    page0, page1 = a.block_table[:2]
    m.deallocate(a)
    # page 0 of a is reused (and cleared) by another request; page 1 stays cached
    while m.free_block_ids[0] != page0:
        m.free_block_ids.rotate(-1)
    m.allocate(Sequence([42, 43]))
    assert m.blocks[page0].token_ids == [] and m.blocks[page1].token_ids == [5, 6, 7, 8]
    b = Sequence([1, 2, 3, 4, 5, 6, 7, 8, 9])
    m.allocate(b)
    assert b.num_cached_tokens == 0 and m.cache_stats()["hits"] == 0  # no reuse after the miss


def test_can_allocate_counts_only_missing_pages():
    m = BlockManager(3, 4)
    a = Sequence([1, 2, 3, 4, 5, 6, 7, 8, 9])  # 3 pages
    assert m.can_allocate(a)
    m.allocate(a)
    assert not m.can_allocate(Sequence([7] * 9))  # 3 fresh pages needed, none free
    b = Sequence([1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
    assert not m.can_allocate(b)  # 2 pages cached, 1 more needed, none free
    m.deallocate(a)
    assert m.can_allocate(b)


def test_trim_to_clears_partial_tail_and_finalises_on_boundary():
    m = BlockManager(8, 4)
    s = Sequence([1, 2, 3])
    m.allocate(s)
    m.ensure_capacity(s, 3 + 6)  # speculative room: 3 pages
    assert len(s.block_table) == 3
    s.token_ids += [4, 5, 6, 7, 8]
    s.num_tokens = 8
    m.trim_to(s, 8)  # confirmed tokens end on a page boundary: page 1 hashed, page 2 released
    assert len(s.block_table) == 2
    tail = m.blocks[s.block_table[1]]
    assert tail.hash != -1 and tail.token_ids == [5, 6, 7, 8]
    assert m.hash_to_block_id[tail.hash] == tail.block_id
    s.token_ids = s.token_ids[:6]
    s.num_tokens = 6
    m.trim_to(s, 6)  # partial tail: its hash is cleared and unregistered
    assert tail.hash == -1 and tail.token_ids == []


def test_register_full_pages_after_device_decoding():
    m = BlockManager(8, 4)
    s = Sequence([1, 2, 3])
    m.allocate(s)
    m.ensure_capacity(s, 11)
    s.token_ids += [4, 5, 6, 7, 8, 9, 10]  # decoded on the device
    s.num_tokens = 10
    m.register_full_pages(s)
    assert [m.blocks[b].token_ids for b in s.block_table[:2]] == [[1, 2, 3, 4], [5, 6, 7, 8]]
    assert m.blocks[s.block_table[2]].hash == -1
    m.deallocate(s)
    t = Sequence([1, 2, 3, 4, 5, 6, 7, 8, 11])
    m.allocate(t)
    assert t.num_cached_tokens == 8


def test_admit_checks_budget_and_reservation():
    sch = Scheduler(4, 10, 6, 4, eos=0)
    seqs = [Sequence([i] * 6) for i in range(3)]
    for s in seqs:
        sch.add_sequence(s)
    # each needs 2 pages for its prompt and 4 pages for its reservation (16 tokens)
    got = sch.admit(4, reserve=lambda s: 16)
    assert got == seqs[:1]  # a second 6-token prompt would exceed the 10-token budget
    assert len(sch.waiting) == 2 and sch.running[0] is seqs[0]
    assert len(seqs[0].block_table) == 4
    sch.finish(seqs[0])
    assert seqs[0].is_finished and not sch.running
    got = sch.admit(4, reserve=lambda s: 8)
    assert got == [seqs[1]]  # budget: 6 + 6 > 10
    assert sch.admit(4, reserve=lambda s: 8) == [seqs[2]]


def test_can_append_asks_for_a_page_exactly_when_needed():
    m = BlockManager(1, 4)
    s = Sequence([1, 2, 3, 4])
    m.allocate(s)
    assert m.can_append(s)  # the 4th token fits the first page; no page needed
    s.append_token(5)
    assert not m.can_append(s)  # the 5th token needs a second page; none is free


def test_preemption_returns_pages_and_requeues():
    sch = Scheduler(2, 64, 2, 4, eos=0)
    a = Sequence([1, 2, 3, 4], SamplingParams(max_tokens=8, ignore_eos=True))
    b = Sequence([5, 6, 7, 8], SamplingParams(max_tokens=8, ignore_eos=True))
    sch.add_sequence(a)
    sch.add_sequence(b)
    scheduled, prefill = sch.schedule()
    assert prefill and scheduled == [a, b]
    sch.postprocess(scheduled, [9, 9])  # both now need a second page; none is free
    scheduled, prefill = sch.schedule()
    assert not prefill
    # b (last in the queue) was preempted so a could grow
    assert scheduled == [a] and sch.waiting[0] is b and not b.block_table
