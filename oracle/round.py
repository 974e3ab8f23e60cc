"""CPU oracle of the round's bookkeeping — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker; the product path never calls it.

  * ``verify_rows`` restates the row building of the reference's graphed
    verify (src/myvllm/engine/model_runner.py:734-774): per sequence, rows
    [last_confirmed, d_1..d_K] at positions n-1..n+K-1 with slot
    table[pos // bs] * bs + pos % bs, context length n + K, and pad rows
    (id 0, position -1, slot -1) up to K+1 rows; inactive slots are all pad
    with context length 0 (the reference's oversized-bucket rows, :768-772).
  * ``commit`` restates SpecLLMEngine._commit (spec_llm_engine.py:249-291)
    on token lists: cap by max_tokens, truncate after eos (unless
    ignore_eos) or at max_model_length, then the finish test.
  * ``draft_rows`` restates the step rows of a model drafter's K decode
    steps (engine/model_runner.py:784-823): step i feeds position n-1+i,
    slot table[pos // bs] * bs + pos % bs; step 0 also re-feeds position
    n-2.  Context length: n+i (keys 0..n-1+i, what the reference's own
    comment at :790-791 and its plain decode, :414, use; its code passes
    n+i+1).
"""

from __future__ import annotations


def verify_rows(histories, drafts, block_tables, block_size: int, K: int, active):
    ids, pos, slots, ctx = [], [], [], []
    for h, d, table, act in zip(histories, drafts, block_tables, active):
        n = len(h)
        live = bool(act) and n > 0
        ctx.append(n + len(d) if live else 0)
        for j in range(K + 1):
            if live and j <= len(d):
                p = n - 1 + j
                ids.append(h[n - 1] if j == 0 else d[j - 1])
                pos.append(p)
                page = table[p // block_size]
                slots.append(-1 if page < 0 else page * block_size + p % block_size)
            else:
                ids.append(0)
                pos.append(-1)
                slots.append(-1)
    return ids, pos, slots, ctx


def commit(history: list[int], prompt_len: int, accepted: list[int], max_tokens: int, eos: int, ignore_eos: bool,
           max_model_length: int | None):
    """Returns (new history, finished)."""
    n = len(history)
    allowed = max(0, max_tokens - (n - prompt_len))
    final = []
    for t in accepted[:allowed]:
        final.append(t)
        reached_eos = not ignore_eos and t == eos
        reached_len = max_model_length is not None and n + len(final) >= max_model_length
        if reached_eos or reached_len:
            break
    new = history[:n] + final
    stop_eos = bool(final) and not ignore_eos and final[-1] == eos
    stop_tokens = len(new) - prompt_len >= max_tokens
    stop_len = max_model_length is not None and len(new) >= max_model_length
    return new, bool(stop_eos or stop_tokens or stop_len)


def draft_rows(histories, block_tables, block_size: int, K: int, active):
    """Returns (ids0, pos0, slot0) of step 0's two rows per sequence and
    (positions, slots, contexts) [K][B] of every step."""
    B = len(histories)
    ids0, pos0, slot0 = [], [], []
    positions = [[-1] * B for _ in range(K)]
    slots = [[-1] * B for _ in range(K)]
    ctx = [[0] * B for _ in range(K)]

    def slot_of(table, p):
        page = table[p // block_size]
        return -1 if page < 0 else page * block_size + p % block_size

    for b, (h, table, act) in enumerate(zip(histories, block_tables, active)):
        n = len(h)
        live = bool(act) and n > 0
        for p in (n - 2, n - 1):
            ok = live and p >= 0
            ids0.append(h[p] if ok else 0)
            pos0.append(p if ok else -1)
            slot0.append(slot_of(table, p) if ok else -1)
        if live:
            for i in range(K):
                p = n - 1 + i
                positions[i][b] = p
                slots[i][b] = slot_of(table, p)
                ctx[i][b] = p + 1
    return ids0, pos0, slot0, positions, slots, ctx
