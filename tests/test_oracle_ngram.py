"""Pins the CPU n-gram oracle (oracle/ngram.py): the bytes.rfind statement
of the reference's lookup against an explicit byte-by-byte search, and
hand-made cases for each branch of the reference's _lookup."""

import json
import os

import numpy as np
import pytest

from oracle import ngram as on

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ngram_cases.json")


@pytest.mark.parametrize("vocab", [3, 40, 300, 70000])
def test_rfind_statement_matches_bruteforce(vocab):
    rng = np.random.default_rng(vocab)
    for _ in range(150):
        L = int(rng.integers(1, 60))
        h = [int(x) for x in rng.integers(0, vocab, size=L)]
        for (k, lo, hi) in [(8, 2, 4), (5, 2, 8), (3, 1, 1)]:
            assert on.lookup(h, k, lo, hi) == on.lookup_bruteforce(h, k, lo, hi), (h, k, lo, hi)


def token_search(history, k, min_n, max_n):
    """Token-level n-gram search without the byte encoding (what the lookup
    would return if misaligned byte hits did not exist)."""
    L = len(history)
    for n in range(min(max_n, L - 1), min_n - 1, -1):
        for i in range(L - 1 - n, -1, -1):
            if history[i:i + n] == history[L - n:]:
                cont = history[i + n:i + n + k]
                if cont:
                    return cont
    return []


def test_misaligned_byte_match_moves_the_search_end():
    # 16843009 = 01 01 01 01 and 16777216 = 01 00 00 00: the 2-gram needle
    # 01 01 01 01 01 01 01 01 first matches at a byte offset inside a token;
    # the reference then only searches left of that offset, which skips the
    # aligned match a token-level search finds
    h = [16843009, 16843009, 16777216, 16777216, 16843009, 16843009]
    assert token_search(h, 3, 2, 3) == [16777216, 16777216, 16843009]
    assert on.lookup(h, 3, 2, 3) == []
    assert on.lookup_bruteforce(h, 3, 2, 3) == []
    h = [256, 257, 16777216, 65793, 1, 65793, 257, 16777216]
    assert token_search(h, 3, 2, 3) == [65793, 1, 65793]
    assert on.lookup(h, 3, 2, 3) == [] == on.lookup_bruteforce(h, 3, 2, 3)
    # without such a straddling hit the byte search and the token search agree
    rng = np.random.default_rng(5)
    for _ in range(200):
        h = [int(x) for x in rng.integers(1 << 24, 1 << 25, size=int(rng.integers(2, 40)))]  # no zero top byte
        h += h[:int(rng.integers(0, 5))]
        assert on.lookup(h, 4, 2, 4) == token_search(h, 4, 2, 4)


def test_edge_cases():
    assert on.lookup([], 4, 2, 8) == []
    assert on.lookup([7], 4, 1, 8) == []                 # L - 1 < min_n
    assert on.lookup([7, 7], 4, 1, 8) == [7]             # match ending just before the last token
    assert on.lookup([1, 2, 3, 1, 2], 8, 2, 8) == [3, 1, 2]   # continuation shorter than k
    assert on.lookup([5, 1, 2, 9, 1, 2], 1, 2, 2) == [9]      # k = 1
    # longest n wins: the 3-gram [1, 2, 3] continues with 4, the 2-gram [2, 3] later with 9
    h = [1, 2, 3, 4, 0, 2, 3, 9, 1, 2, 3]
    assert on.lookup(h, 1, 2, 3) == [4]
    assert on.lookup(h, 1, 2, 2) == [9]


def test_golden_cases():
    for c in json.load(open(GOLDEN)):
        assert on.lookup(c["history"], c["k"], c["min_n"], c["max_n"]) == c["expected"], c
