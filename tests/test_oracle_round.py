"""Pins the round-bookkeeping oracle (oracle/round.py) with closed-form
cases of the reference's _commit and verify-row layout, and the host
BlockManager's speculative capacity API."""

from naivllm_amd.engine.block_manager import BlockManager
from naivllm_amd.engine.sequence import Sequence
from oracle import round as orr


def test_verify_rows_layout():
    # n = 5 tokens, 2 drafts, K = 3: rows at positions 4, 5, 6 then one pad row
    ids, pos, slots, ctx = orr.verify_rows([[1, 2, 3, 4, 5]], [[7, 8]], [[3, 9]], 4, 3, [1])
    assert ids == [5, 7, 8, 0]
    assert pos == [4, 5, 6, -1]
    assert slots == [9 * 4 + 0, 9 * 4 + 1, 9 * 4 + 2, -1]   # positions 4..6 live in page 1 -> id 9
    assert ctx == [7]
    # inactive slot: all pad, context 0
    ids, pos, slots, ctx = orr.verify_rows([[1, 2]], [[3]], [[0]], 4, 1, [0])
    assert (ids, pos, slots, ctx) == ([0, 0], [-1, -1], [-1, -1], [0])


def test_commit_caps_and_stops():
    h = [9, 9, 9, 1, 2]  # prompt of 3, 2 completion tokens so far
    # plenty of room: everything accepted is appended
    assert orr.commit(h, 3, [5, 6, 7], 10, eos=0, ignore_eos=False, max_model_length=None) == (h + [5, 6, 7], False)
    # max_tokens: only 1 more completion token allowed, and the sequence finishes
    assert orr.commit(h, 3, [5, 6, 7], 3, eos=0, ignore_eos=False, max_model_length=None) == (h + [5], True)
    # eos stops after itself ...
    assert orr.commit(h, 3, [5, 0, 7], 10, eos=0, ignore_eos=False, max_model_length=None) == (h + [5, 0], True)
    # ... unless ignored
    assert orr.commit(h, 3, [5, 0, 7], 10, eos=0, ignore_eos=True, max_model_length=None) == (h + [5, 0, 7], False)
    # max_model_length: length 7 reached after two tokens
    assert orr.commit(h, 3, [5, 6, 7], 10, eos=0, ignore_eos=False, max_model_length=7) == (h + [5, 6], True)
    # already at max_tokens: nothing appended, finished
    assert orr.commit(h, 3, [5], 2, eos=0, ignore_eos=False, max_model_length=None) == (h, True)


def test_block_manager_speculative_capacity_and_trim():
    bm = BlockManager(num_blocks=6, block_size=4)
    s = Sequence([1, 2, 3, 4, 5])
    bm.allocate(s)
    assert len(s.block_table) == 2
    assert bm.can_ensure_capacity(s, 5 + 8)         # needs 2 more pages, 4 free
    bm.ensure_capacity(s, 5 + 8)
    assert len(s.block_table) == 4 and len(bm.free_block_ids) == 2
    assert not bm.can_ensure_capacity(s, 40)
    bm.trim_to(s, 6)                                 # back to ceil(6/4) = 2 pages
    assert len(s.block_table) == 2 and len(bm.free_block_ids) == 4
    s.append_token(6)
    bm.rollback(s, 1)                                # the reference's rollback test (tests/test_block_manager.py:43-53)
    assert s.token_ids == [1, 2, 3, 4, 5] and len(s.block_table) == 2
    bm.deallocate(s)
    assert len(bm.free_block_ids) == 6 and not s.block_table


def test_draft_rows_layout():
    # n = 5 tokens, block size 4, table [3, 9]: step 0 feeds positions 3 and 4, steps 1..2 positions 5, 6
    ids0, pos0, slot0, pos, slots, ctx = orr.draft_rows([[1, 2, 3, 4, 5], [7]], [[3, 9], [2, -1]], 4, 3, [1, 1])
    assert ids0 == [4, 5, 0, 7] and pos0 == [3, 4, -1, 0]
    assert slot0 == [3 * 4 + 3, 9 * 4 + 0, -1, 2 * 4 + 0]
    assert pos == [[4, 0], [5, 1], [6, 2]]
    assert slots == [[36, 8], [37, 9], [38, 10]]
    assert ctx == [[5, 1], [6, 2], [7, 3]]    # keys up to the fed position
    # inactive: pads, context 0
    ids0, pos0, slot0, pos, slots, ctx = orr.draft_rows([[1, 2, 3]], [[0]], 4, 2, [0])
    assert (ids0, pos0, slot0) == ([0, 0], [-1, -1], [-1, -1]) and pos == [[-1], [-1]] and ctx == [[0], [0]]
