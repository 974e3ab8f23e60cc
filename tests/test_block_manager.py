"""Host bookkeeping of pages and requests on the CPU.

Behaviours of src/myvllm/engine/block_manager.py (:58-300) and
src/myvllm/engine/scheduler.py (:25-98) that the reference's callers rely
on: page arithmetic at page boundaries, prefix-cache reuse after release,
pinning, rollback, the max_tokens stop, admission and preemption; plus this
build's page accounting for reservations and device-written pages."""

import pytest

from naivllm_amd.engine.block_manager import BlockManager
from naivllm_amd.engine.scheduler import Scheduler
from naivllm_amd.engine.sequence import Sequence, SequenceStatus
from naivllm_amd.sampling_parameters import SamplingParams


# ---- page arithmetic ---------------------------------------------------------
@pytest.mark.parametrize("bs,n,pages,last", [(8, 16, 2, 8), (8, 17, 3, 1), (8, 8, 1, 8), (256, 1248, 5, 224)])
def test_page_count_and_last_page_fill(bs, n, pages, last):
    s = Sequence(list(range(100, 100 + n)))
    s.block_size = bs
    assert s.num_blocks == pages and s.last_block_num_tokens == last
    assert s.block(pages - 1) == list(range(100 + (pages - 1) * bs, 100 + n))
    assert sum(len(s.block(i)) for i in range(pages)) == n


def test_released_page_is_found_again_by_a_sharing_prompt():
    m = BlockManager(num_blocks=6, block_size=8)
    doc = list(range(1, 17))  # two full pages
    a = Sequence(doc + [50, 51])
    m.allocate(a)
    p0, p1 = a.block_table[:2]
    m.deallocate(a)
    assert set(m.free_block_ids) == set(range(6))  # every page back in the pool
    b = Sequence(doc[:8] + [7] * 8 + [60])  # shares page 0 only
    m.allocate(b)
    assert b.block_table[0] == p0 and b.block_table[1] != p1
    assert b.num_cached_tokens == 8
    assert m.blocks[p0].ref_count == 1 and m.blocks[p0].token_ids == doc[:8]
    stats = m.cache_stats()
    assert stats["hits"] == 1 and stats["misses"] == 3 + 2


def test_pins_hold_pages_until_unpinned():
    m = BlockManager(num_blocks=5, block_size=4)
    a = Sequence([9, 8, 7, 6, 5, 4, 3, 2, 1])
    m.allocate(a)
    held = a.block_table[:2]
    m.deallocate(a)
    assert m.pin_prefix([9, 8, 7, 6, 5, 4, 3, 2]) == 8
    assert m.pin_prefix([9, 8, 7, 6]) == 4  # a second pin of the first page
    assert all(b in m.used_block_ids and b not in m.free_block_ids for b in held)
    assert m.cache_stats()["pinned_blocks"] == 2 and m.cache_stats()["free_blocks"] == 3
    # a request needing every page cannot take the pinned ones
    assert not m.can_allocate(Sequence([0] * 17))
    m.unpin_all()
    assert all(b in m.free_block_ids for b in held) and m.blocks[held[0]].ref_count == 0
    assert m.can_allocate(Sequence([0] * 17))


def test_rollback_returns_pages_of_removed_tokens():
    m = BlockManager(num_blocks=6, block_size=4)
    s = Sequence([1, 2, 3])
    m.allocate(s)
    for t in range(4, 11):  # decode 7 tokens, pages on demand
        s.append_token(t)
        m.append(s)
    assert len(s.block_table) == 3 and len(m.free_block_ids) == 3
    m.rollback(s, 6)  # back to 4 tokens: one full page
    assert s.token_ids == [1, 2, 3, 4] and s.last_token == 4 and s.num_tokens == 4
    assert len(s.block_table) == 1 and len(m.free_block_ids) == 5
    with pytest.raises(ValueError):
        m.rollback(s, 2)  # only one completion token is left


@pytest.mark.parametrize("max_tokens", [1, 2, 5])
def test_decode_stops_at_exactly_max_tokens(max_tokens):
    sch = Scheduler(2, 64, 8, 4, eos=99)
    s = Sequence([1, 2, 3], SamplingParams(max_tokens=max_tokens, ignore_eos=True))
    sch.add_sequence(s)
    steps = 0
    while not sch.is_finished():
        seqs, _ = sch.schedule()
        sch.postprocess(seqs, [99] * len(seqs))  # EOS is ignored
        steps += 1
    assert steps == max_tokens and s.completion_token_ids == [99] * max_tokens
    assert s.is_finished and not s.block_table and len(sch.block_manager.free_block_ids) == 8


def test_eos_and_model_length_stop():
    sch = Scheduler(4, 64, 8, 4, eos=7)
    a = Sequence([1, 2], SamplingParams(max_tokens=10))
    b = Sequence([1, 2], SamplingParams(max_tokens=10, ignore_eos=True, max_model_length=4))
    sch.add_sequence(a)
    sch.add_sequence(b)
    seqs, prefill = sch.schedule()
    assert prefill and seqs == [a, b]
    sch.postprocess(seqs, [7, 7])
    assert a.is_finished and not b.is_finished
    seqs, prefill = sch.schedule()
    assert not prefill and seqs == [b]
    sch.postprocess(seqs, [5])
    assert b.is_finished and b.num_tokens == 4 and sch.is_finished()


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


# ---- page accounting for reservations and device-written pages ---------------
def test_can_allocate_counts_cached_hits_taken_from_the_free_queue():
    m = BlockManager(num_blocks=4, block_size=4)
    a = Sequence(list(range(1, 14)))  # 3 full pages + 1
    m.allocate(a)
    m.deallocate(a)  # 4 free pages, 3 of them cached
    b = Sequence(list(range(1, 13)) + list(range(20, 29)))  # 3 hits + 3 fresh pages
    assert m.free_pages_needed(b) == 6
    assert not m.can_allocate(b)  # taking the hits leaves 1 free page for 3
    c = Sequence(list(range(1, 13)) + [30])  # 3 hits + 1 fresh page
    assert m.can_allocate(c)
    m.allocate(c)
    assert c.num_cached_tokens == 12 and not m.free_block_ids
    # a held hit costs no free page: a second sharer needs only its own tail
    d = Sequence(list(range(1, 13)) + [31])
    assert m.free_pages_needed(d) == 1 and not m.can_allocate(d)


def test_failed_reservation_leaves_no_registered_pages():
    sch = Scheduler(4, 1000, 4, 4, eos=0)
    bm = sch.block_manager
    blocker = Sequence([5] * 8)
    bm.allocate(blocker)  # holds 2 of the 4 pages
    s = Sequence(list(range(1, 10)))  # 3 pages of prompt, 2 of them full
    sch.add_sequence(s)
    assert sch.admit(4, reserve=lambda q: 12) == []  # 3 pages needed, 2 free
    assert sch.waiting[0] is s and not s.block_table and len(bm.free_block_ids) == 2
    bm.deallocate(blocker)
    assert sch.admit(4, reserve=lambda q: 12) == [s]
    assert s.num_cached_tokens == 0  # nothing it never computed was served from the cache
    assert len(s.block_table) == 3


def test_register_full_pages_skips_the_page_of_the_last_token():
    # the device round writes a token's KV one round after committing it, so a
    # sequence ending on a page boundary has no KV for its last token
    m = BlockManager(8, 4)
    s = Sequence([1, 2, 3])
    m.allocate(s)
    m.ensure_capacity(s, 12)
    s.token_ids += [4, 5, 6, 7, 8]
    s.num_tokens = 8
    m.register_full_pages(s)
    assert m.blocks[s.block_table[0]].token_ids == [1, 2, 3, 4]
    assert m.blocks[s.block_table[1]].hash == -1  # ends at the last token
    m.deallocate(s)
    t = Sequence([1, 2, 3, 4, 5, 6, 7, 8, 9, 10])  # extends s
    m.allocate(t)
    assert t.num_cached_tokens == 4
    # right after prefill (prompt + first token on a boundary) likewise
    u = Sequence([11, 12, 13])
    m.allocate(u)
    u.append_token(14)
    m.register_full_pages(u)
    assert m.blocks[u.block_table[0]].hash == -1


def test_decode_step_preempts_from_the_back_until_pages_fit():
    sch = Scheduler(4, 64, 4, 4, eos=0)
    seqs = [Sequence([i] * 4, SamplingParams(max_tokens=8, ignore_eos=True)) for i in (1, 2, 3)]
    for s in seqs:
        sch.add_sequence(s)
    got, prefill = sch.schedule()
    assert prefill and got == seqs and len(sch.block_manager.free_block_ids) == 1
    sch.postprocess(got, [9, 9, 9])  # each now needs a second page; one is free
    got, prefill = sch.schedule()
    # 3 pages wanted, 1 free: preempting the last sequence frees its page and
    # drops its demand, after which the first two fit
    assert not prefill and got == seqs[:2]
    assert list(sch.waiting) == [seqs[2]] and seqs[2].status == SequenceStatus.WAITING
    assert not seqs[2].block_table
    assert list(sch.running) == seqs[:2] and all(len(s.block_table) == 2 for s in seqs[:2])
    sch.postprocess(got, [9, 9])
    for _ in range(3):  # 3 more tokens fit the second pages
        got, _ = sch.schedule()
        assert got == seqs[:2]
        sch.postprocess(got, [9, 9])
    got, _ = sch.schedule()  # both need a third page, none is free: b goes
    assert got == [seqs[0]] and list(sch.waiting) == [seqs[1], seqs[2]]
