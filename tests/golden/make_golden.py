"""Writes the small golden fixtures under tests/golden/.

Expected values come from brute-force pure-Python loops written from the
mathematics (not from the oracle under test), on inputs from the seeded
generator in naivllm_amd.utils.synth; inputs are stored in the fixture too,
so the fixture alone pins the oracle and the GPU path.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import math
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from naivllm_amd.utils import synth  # noqa: E402


def brute_attention(case):
    """out[r][h][d] = sum_j softmax_j(scale * <q[r][h], k_j>) v_j[d] over the
    keys j <= pos[r] of row r's sequence whose page is mapped; kv head h // G."""
    q, kc, vc = case["q"], case["k_cache"], case["v_cache"]
    bt, ctx, cu, pos = case["block_tables"], case["context_lens"], case["cu_seqlens_q"], case["positions"]
    H, Hkv, D, bs, scale = case["num_heads"], case["num_kv_heads"], case["head_dim"], case["block_size"], case["scale"]
    G = H // Hkv
    out = [[[0.0] * D for _ in range(H)] for _ in range(len(q))]
    for b in range(len(ctx)):
        for r in range(cu[b], cu[b + 1]):
            if pos[r] < 0:
                continue
            for h in range(H):
                kvh = h // G
                keys = [j for j in range(min(ctx[b], len(bt[b]) * bs))
                        if j <= pos[r] and bt[b][j // bs] >= 0]
                if not keys:
                    continue
                scores = []
                for j in keys:
                    row = kc[bt[b][j // bs]][j % bs][kvh]
                    scores.append(scale * sum(q[r][h][d] * row[d] for d in range(D)))
                mx = max(scores)
                w = [math.exp(s - mx) for s in scores]
                z = sum(w)
                for d in range(D):
                    out[r][h][d] = sum(w[i] * vc[bt[b][j // bs]][j % bs][kvh][d] for i, j in enumerate(keys)) / z
    return out


def attention_tiny():
    # two sequences with ragged query counts, a hole in the block table and
    # an inert pad row; head_dim 4, GQA group 2, 4-token pages
    vb = synth.verify_batch(11, [11, 6], [3, 2], num_heads=4, num_kv_heads=2, head_dim=4, block_size=4,
                            num_blocks=7, max_blocks=4, dtype="f32", pad_rows=[0, 1])
    bt = vb.block_tables.copy()
    bt[0, 1] = -1  # unmapped middle page: keys 4..7 of sequence 0 are skipped
    case = dict(
        q=vb.q.tolist(), k_cache=vb.k_cache.tolist(), v_cache=vb.v_cache.tolist(),
        block_tables=bt.tolist(), context_lens=vb.context_lens.tolist(),
        cu_seqlens_q=vb.cu_seqlens_q.tolist(), positions=vb.positions.tolist(),
        num_heads=4, num_kv_heads=2, head_dim=4, block_size=4, scale=0.5,
    )
    case["expected"] = brute_attention(case)
    return case


def _be_bytes(tokens):
    return b"".join(int(t).to_bytes(4, "big") for t in tokens)


def brute_ngram(history, k, min_n, max_n):
    """The reference's lookup (drafters.py:63-83) by explicit byte scans:
    right-most match of the suffix's big-endian bytes ending at or before
    byte 4*(L-1); a hit inside a token restarts the scan left of it."""
    L = len(history)
    hay = _be_bytes(history)
    for n in range(min(max_n, L - 1), min_n - 1, -1):
        needle = hay[4 * (L - n):]
        end = 4 * (L - 1)
        while True:
            idx = -1
            for i in range(end - len(needle), -1, -1):
                if hay[i:i + len(needle)] == needle:
                    idx = i
                    break
            if idx == -1 or idx % 4 == 0:
                break
            end = idx
        if idx != -1:
            cont = history[idx // 4 + n: idx // 4 + n + k]
            if cont:
                return cont
    return []


def ngram_cases():
    cases = []
    fixed = [
        ([16843009, 16843009, 16777216, 16777216, 16843009, 16843009], 3, 2, 3),  # straddling hit
        ([256, 257, 16777216, 65793, 1, 65793, 257, 16777216], 3, 2, 3),
        ([256, 512, 1, 2, 3, 256, 512], 2, 2, 2),
        ([1, 2, 3, 1, 2], 8, 2, 8),
        ([7, 7], 4, 1, 8),
        ([7], 4, 1, 8),
        ([], 4, 2, 8),
        ([1, 2, 3, 4, 0, 2, 3, 9, 1, 2, 3], 1, 2, 3),
    ]
    for h, k, lo, hi in fixed:
        cases.append(dict(history=h, k=k, min_n=lo, max_n=hi))
    for seed in range(12):
        vocab = [4, 50, 151936][seed % 3]
        L = 20 + 7 * seed
        h = [int(x) for x in synth.randint(seed, 40, L, 0, vocab)]
        cases.append(dict(history=h, k=8, min_n=2, max_n=4 + seed % 5))
    for c in cases:
        c["expected"] = brute_ngram(c["history"], c["k"], c["min_n"], c["max_n"])
    return cases


def main():
    with open(os.path.join(HERE, "attention_tiny.json"), "w") as f:
        json.dump(attention_tiny(), f)
    print("wrote attention_tiny.json")
    with open(os.path.join(HERE, "ngram_cases.json"), "w") as f:
        json.dump(ngram_cases(), f)
    print("wrote ngram_cases.json")


if __name__ == "__main__":
    main()
