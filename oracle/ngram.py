"""CPU oracle of the n-gram (prompt-lookup) drafter — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker; the product path never calls it.

``lookup`` restates NgramDrafter._lookup (src/myvllm/spec_engine/
drafters.py:63-83): for n = min(max_n, L-1) down to min_n, encode the
history as big-endian uint32 bytes and search the last n tokens' bytes with
CPython's ``bytes.rfind`` over haystack[0 : 4*(L-1)].  A hit at a byte
offset that is not a multiple of 4 (a match straddling token boundaries)
moves the search end to that offset and searches again — so aligned matches
overlapping a misaligned one to its right are skipped, exactly as in the
reference.  The first aligned hit yields history[idx/4 + n : +k], which is
never empty because the match ends before the last token.

``lookup_bruteforce`` is an independent statement of the same function that
never calls ``rfind``: it scans byte offsets right to left and compares byte
by byte; the tests pin ``lookup`` against it (and both against hand-made
adversarial cases).
"""

from __future__ import annotations

import numpy as np


def encode(tokens) -> bytes:
    return np.asarray(tokens, dtype=">u4").tobytes()


def lookup(history, k: int, min_n: int, max_n: int) -> list[int]:
    history = [int(t) for t in history]
    L = len(history)
    hay = encode(history)
    for n in range(min(max_n, L - 1), min_n - 1, -1):
        needle = encode(history[L - n:])
        end = 4 * (L - 1)
        while True:
            idx = hay.rfind(needle, 0, end)
            if idx == -1 or idx % 4 == 0:
                break
            end = idx
        if idx != -1:
            start = idx // 4 + n
            cont = history[start:start + k]
            if cont:
                return cont
    return []


def _rfind_bytes(hay: bytes, needle: bytes, end: int) -> int:
    """Largest i with i + len(needle) <= end and hay[i:i+len] == needle, by
    explicit comparison (no library search)."""
    n = len(needle)
    i = end - n
    while i >= 0:
        j = 0
        while j < n and hay[i + j] == needle[j]:
            j += 1
        if j == n:
            return i
        i -= 1
    return -1


def lookup_bruteforce(history, k: int, min_n: int, max_n: int) -> list[int]:
    history = [int(t) for t in history]
    L = len(history)
    hay = encode(history)
    for n in range(min(max_n, L - 1), min_n - 1, -1):
        needle = hay[4 * (L - n):]
        end = 4 * (L - 1)
        idx = _rfind_bytes(hay, needle, end)
        while idx != -1 and idx % 4 != 0:
            idx = _rfind_bytes(hay, needle, idx)
        if idx != -1:
            start = idx // 4 + n
            cont = history[start:start + k]
            if cont:
                return cont
    return []


def draft(histories, k: int, min_n: int, max_n: int) -> list[list[int]]:
    """NgramDrafter.draft's token choice (drafters.py:46-61) for a batch."""
    return [lookup(h, k, min_n, max_n) for h in histories]
