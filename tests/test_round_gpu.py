"""The device-resident verification round: its bookkeeping kernels against
the CPU oracle, one whole round against a host restatement of the
reference's round (n-gram lookup, greedy walk, commit) on the logits the
GPU forward produced, and end-to-end properties: greedy speculative
decoding emits exactly the tokens of plain greedy decoding through the same
forward, and graph replay equals eager execution."""

import numpy as np
import pytest
import torch

from naivllm_amd.engine.verify_round import commit, prepare_verify
from naivllm_amd.layers.qwen3 import Qwen3Config
from naivllm_amd.sampling_parameters import SamplingParams
from naivllm_amd.spec_engine.spec_llm_engine import SpecLLMEngine
from naivllm_amd.utils import synth
from oracle import accept as oa
from oracle import ngram as on
from oracle import round as orr

pytestmark = pytest.mark.gpu

TINY = Qwen3Config(vocab_size=2048, hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64,
                   intermediate_size=512, max_position=4096)


def i32(x):
    return torch.tensor(x, dtype=torch.int32, device="cuda")


def test_prepare_and_commit_kernels_match_oracle():
    print("case: prepare/commit kernels", flush=True)
    B, K, S, bs, MB = 6, 4, 64, 8, 8
    hists = [[int(x) for x in synth.randint(b, 80, L, 0, 50)] for b, L in enumerate([10, 1, 31, 0, 17, 40])]
    drafts = [[int(x) for x in synth.randint(b, 81, k, 0, 50)] for b, k in enumerate([4, 2, 0, 3, 4, 1])]
    active = [1, 1, 1, 1, 0, 1]
    tables = [[int(x) for x in synth.randperm(b, 82, 64)[:MB]] for b in range(B)]
    tables[2][3] = -1
    H = torch.zeros(B, S, dtype=torch.int32)
    for b, h in enumerate(hists):
        H[b, :len(h)] = torch.tensor(h, dtype=torch.int32)
    D = torch.zeros(B, K, dtype=torch.int32)
    for b, d in enumerate(drafts):
        D[b, :len(d)] = torch.tensor(d, dtype=torch.int32)
    H, D = H.cuda(), D.cuda()
    hl, nd, act, bt = i32([len(h) for h in hists]), i32([len(d) for d in drafts]), i32(active), i32(tables)
    ids = torch.empty(B * (K + 1), dtype=torch.int64, device="cuda")
    pos, slots, ctx = torch.empty_like(ids), torch.empty_like(ids), torch.empty(B, dtype=torch.int64, device="cuda")
    prepare_verify(H, hl, D, nd, bt, bs, act, K, ids, pos, slots, ctx)
    want = orr.verify_rows(hists, drafts, tables, bs, K, active)
    assert (ids.tolist(), pos.tolist(), slots.tolist(), ctx.tolist()) == want

    # commit: accepted lists of various lengths against the oracle
    acc = [[5, 6, 7], [9], [1, 2, 3, 4, 5], [0, 1], [3], [2, 0, 4]]
    T = torch.zeros(B, K + 1, dtype=torch.int32)
    for b, a in enumerate(acc):
        T[b, :len(a)] = torch.tensor(a, dtype=torch.int32)
    prompt = [5, 0, 20, 0, 10, 38]
    maxt = [10, 3, 13, 5, 10, 4]
    maxlen = [0, 0, 33, 0, 0, 0]
    ign = [0, 1, 0, 0, 0, 0]
    committed = torch.zeros(B, dtype=torch.int32, device="cuda")
    commit(T.cuda(), i32([len(a) for a in acc]), nd, H, hl, i32(prompt), i32(maxt), i32(maxlen), i32(ign), 0, act,
           committed, K)
    Hh, hlh, acth = H.cpu(), hl.cpu().tolist(), act.cpu().tolist()
    for b in range(B):
        if not active[b]:
            assert hlh[b] == len(hists[b]) and acth[b] == 0
            continue
        new, fin = orr.commit(hists[b], prompt[b], acc[b], maxt[b], 0, bool(ign[b]), maxlen[b] or None)
        assert Hh[b, :hlh[b]].tolist() == new, b
        assert acth[b] == int(not fin), b


def test_one_round_matches_host_restatement():
    # one eager round: drafts, acceptance and commit against the oracle's
    # lookup / greedy walk / _commit applied to the logits the forward produced
    print("case: round vs host restatement", flush=True)
    eng = SpecLLMEngine(dict(model_config=TINY, num_speculative_tokens=4, ngram_min_size=1, ngram_max_size=3,
                             max_num_sequences=4, max_model_length=256, block_size=16, enforce_eager=True))
    r = eng.round
    B, K = 4, 4
    rng = np.random.default_rng(0)
    hists = []
    for b in range(B):
        span = [int(x) for x in rng.integers(0, 60, 12)]
        hists.append((span * 4)[: 30 + 5 * b])
    for b, h in enumerate(hists):
        from naivllm_amd.engine.sequence import Sequence
        s = Sequence(h)
        eng.block_manager.allocate(s)
        eng.block_manager.ensure_capacity(s, len(h) + 64)
        eng._prefill([s])
        r.history[b, :len(h)] = torch.tensor(h, dtype=torch.int32, device="cuda")
        r.hist_len[b] = len(h)
        r.prompt_len[b] = len(h) - 2
        r.max_tokens[b] = 100
        r.max_len[b] = 256
        r.ignore_eos[b] = 1
        r.active[b] = 1
        r.block_tables[b].fill_(-1)
        r.block_tables[b, :len(s.block_table)] = torch.tensor(s.block_table, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    r.body(B)
    torch.cuda.synchronize()
    drafts = [r.drafts[b, :int(r.num_drafts[b])].tolist() for b in range(B)]
    assert drafts == on.draft(hists, K, 1, 3)
    logits = r.logits[:B * (K + 1)].float().cpu().numpy()
    accepted = oa.greedy_round(drafts, logits, K + 1)
    for b in range(B):
        new, fin = orr.commit(hists[b], len(hists[b]) - 2, accepted[b], 100, -1, True, 256)
        assert r.history[b, :int(r.hist_len[b])].tolist() == new
        assert int(r.committed[b]) == len(accepted[b])


# K = 40: 41 verify rows per sequence (two query heads per kv head: 82 rows, served one head at a
# time by the attention), acceptance walks past lane 32
@pytest.mark.parametrize("block_size,K", [(16, 6), (64, 6), (16, 40)])
def test_greedy_spec_equals_plain_decode_and_graph_equals_eager(block_size, K):
    print(f"case: e2e spec==plain bs={block_size} K={K}", flush=True)
    rng = np.random.default_rng(1)
    prompts = []
    for b in range(3):
        spans = [[int(x) for x in rng.integers(0, 2048, 10)] for _ in range(4)]
        prompts.append([t for i in range(12) for t in spans[i % 4]] + spans[0][:3])
    sp = SamplingParams(temperature=0.0, max_tokens=40, ignore_eos=True)
    base = dict(model_config=TINY, num_speculative_tokens=K, ngram_min_size=2, ngram_max_size=4,
                max_num_sequences=4, max_model_length=512, block_size=block_size, seed=3)
    out = {}
    for name, extra in [("spec", {}), ("plain", {"spec_method": "none"}), ("spec_eager", {"enforce_eager": True})]:
        eng = SpecLLMEngine({**base, **extra})
        res = eng.generate(prompts, sp)
        out[name] = [o["token_ids"] for o in res["outputs"]]
        m = res["metrics"]
        print(name, m["rounds"], m["spec_decoding"], flush=True)
        # rounds are enqueued ahead of their reports: every launched round is
        # read back and counted once, and the decode tokens are exactly the
        # tokens after each sequence's prefill token
        assert m["rounds"] == m["spec_decoding"]["rounds"]
        assert m["decode_tokens"] == sum(len(t) for t in out[name]) - len(prompts)
        del eng
        torch.cuda.empty_cache()
    assert all(len(x) == 40 for x in out["spec"])
    assert out["spec"] == out["spec_eager"]
    assert out["spec"] == out["plain"]
