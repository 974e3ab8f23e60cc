"""GPU parity of the n-gram drafter kernel against the CPU oracle (byte-exact
reproduction of the reference's bytes.rfind lookup)."""

import json
import os

import numpy as np
import pytest
import torch

from naivllm_amd.engine.sequence import Sequence
from naivllm_amd.spec_engine import NgramDrafter
from naivllm_amd.spec_engine.drafters import ngram_draft
from naivllm_amd.utils import synth
from oracle import ngram as on

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ngram_cases.json")


def run(histories, k, lo, hi, stride=None):
    B = len(histories)
    S = stride or max(1, max(len(h) for h in histories))
    hist = torch.full((B, S), -7, dtype=torch.int32)
    for b, h in enumerate(histories):
        if h:
            hist[b, :len(h)] = torch.tensor(np.asarray(h, dtype=np.uint32).view(np.int32))
    lens = torch.tensor([len(h) for h in histories], dtype=torch.int32)
    d, n = ngram_draft(hist.cuda(), lens.cuda(), k, lo, hi)
    d = d.cpu().numpy().view(np.uint32)
    return [[int(x) for x in d[b, :m]] for b, m in enumerate(n.cpu().tolist())]


def test_golden_cases():
    print("case: ngram golden", flush=True)
    cases = json.load(open(GOLDEN))
    for c in cases:
        assert run([c["history"]], c["k"], c["min_n"], c["max_n"]) == [c["expected"]], c


@pytest.mark.parametrize("vocab", [2, 5, 300, 151936])
def test_random_batches_match_oracle(vocab):
    print(f"case: ngram random vocab={vocab}", flush=True)
    for rep in range(6):
        B = 16
        lens = [int(x) for x in synth.randint(rep, 70 + vocab % 97, B, 0, 300)]
        lens[0], lens[1] = 0, 1
        hs = [[int(x) for x in synth.randint(rep * 100 + b, 71, L, 0, vocab)] for b, L in enumerate(lens)]
        for (k, lo, hi) in [(8, 2, 4), (5, 1, 8)]:
            assert run(hs, k, lo, hi) == on.draft(hs, k, lo, hi)


def test_straddling_byte_hits():
    # token values whose bytes are 0/1 make hits at byte offsets inside tokens common
    print("case: ngram straddling", flush=True)
    vals = np.array([0x01010101, 0x00010101, 0x01010100, 0x00000101, 0x01000000, 0x00000001, 256, 512],
                    dtype=np.int64)
    hs = []
    for rep in range(64):
        L = 4 + rep % 40
        hs.append([int(vals[i]) for i in synth.randint(rep, 72, L, 0, len(vals))])
    assert run(hs, 3, 2, 3) == on.draft(hs, 3, 2, 3)
    assert run(hs, 8, 1, 6) == on.draft(hs, 8, 1, 6)


def test_long_history_reads_global_memory():
    # histories longer than the kernel's LDS copy (12288 tokens)
    print("case: ngram long", flush=True)
    L = 20000
    h = [int(x) for x in synth.randint(8, 73, L, 0, 50000)]
    h[-3:] = h[1000:1003]      # plant a 3-gram match early in the history
    h2 = [int(x) for x in synth.randint(9, 73, 15000, 0, 3)]
    assert run([h, h2], 8, 2, 4) == on.draft([h, h2], 8, 2, 4)


def test_drop_in_draft_appends_to_sequences():
    print("case: ngram drop-in", flush=True)
    prompt = [5, 6, 7, 8, 9, 1, 2, 3, 5, 6, 7]
    seqs = [Sequence(prompt), Sequence([1, 2]), Sequence([4, 4, 4, 4])]
    drafter = NgramDrafter(num_speculative_tokens=3, min_ngram_size=2, max_ngram_size=4)
    drafts, rows = drafter.draft(seqs)
    assert rows == [None, None, None]
    assert drafts == [on.lookup(prompt, 3, 2, 4), [], on.lookup([4, 4, 4, 4], 3, 2, 4)]
    assert drafts[0] == [8, 9, 1]
    assert seqs[0].draft_tokens == [8, 9, 1] and seqs[0].token_ids == prompt + [8, 9, 1]
    assert seqs[0].num_tokens == len(prompt) + 3 and seqs[0].last_token == 1
    assert seqs[1].draft_tokens == [] and seqs[1].num_tokens == 2
