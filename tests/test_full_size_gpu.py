"""Parity at the BASELINE configurations' full sizes.

  * config 4: verify attention at the Qwen3-8B layer shape (B=16, 32Q/8KV,
    contexts U[16k, 32k], 256-token pages in a seeded permuted pool, K=8)
    through the key-split kernel, against the oracle on a seeded subset of
    sequences (the shortest, the longest and two others: every row of each);
  * config 3: the greedy n-gram round of a random-init Qwen3-0.6B (28
    layers, vocab 151936) on the config-3 prompts at b1 and b8: one eager
    round against the host restatement (oracle n-gram lookup, greedy walk,
    commit) on the logits the forward produced; then 48 greedy tokens where
    speculative decoding must emit exactly plain greedy decoding's tokens
    and the graphed round exactly the eager round's;
  * config 5: one stochastic hybrid round of a random-init Qwen3-0.6B
    drafter feeding a random-init Qwen3-8B target at T = 1.0, b1 and b8,
    against the oracle's sampler, acceptance and commit on that round's own
    logits and random draws.
"""

import numpy as np
import pytest
import torch

from naivllm_amd.engine.sequence import Sequence
from naivllm_amd.layers.attention import paged_attention_verify, verify_attention_plan
from naivllm_amd.layers.qwen3 import Qwen3Config
from naivllm_amd.sampling_parameters import SamplingParams
from naivllm_amd.spec_engine.spec_llm_engine import SpecLLMEngine
from naivllm_amd.utils import synth
from oracle import accept as oa
from oracle import attention as ora
from oracle import ngram as on
from oracle import round as orr
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu


def test_config4_attention_full_size():
    B, H, Hkv, D, bs, R = 16, 32, 8, 128, 256, 9
    seed = 4
    ctx = [int(x) for x in synth.randint(seed, 7, B, 16384, 32769)]
    pages = [(c + bs - 1) // bs for c in ctx]
    nb = sum(pages) + 37
    mb = max(pages)
    print(f"case: config4 attention B=16 32Q/8KV ctx {min(ctx)}..{max(ctx)} pool {nb} pages", flush=True)
    kernel, splits = verify_attention_plan(B, H, Hkv, D, bs, mb, R, torch.bfloat16)
    assert kernel == "key-split" and splits >= 2, (kernel, splits)
    perm = synth.randperm(seed, 1, nb)
    bt = np.full((B, mb), -1, dtype=np.int32)
    off = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    g = torch.Generator(device="cuda").manual_seed(seed)
    kc = torch.randn(nb, bs, Hkv, D, generator=g, device="cuda", dtype=torch.bfloat16)
    vc = torch.randn(nb, bs, Hkv, D, generator=g, device="cuda", dtype=torch.bfloat16)
    q = torch.randn(B * R, H, D, generator=g, device="cuda", dtype=torch.bfloat16)
    pos = np.concatenate([np.arange(c - R, c) for c in ctx])
    out = paged_attention_verify(q, kc, vc, torch.from_numpy(bt).cuda(), torch.tensor(ctx, device="cuda"),
                                 torch.arange(0, B * R + 1, R, dtype=torch.int32, device="cuda"),
                                 torch.from_numpy(pos).cuda(), 1 / np.sqrt(D), H, Hkv, D, bs, 16, max_q_len=R)
    torch.cuda.synchronize()
    order = np.argsort(ctx)
    subset = sorted({int(order[0]), int(order[-1]), int(synth.randint(seed, 8, 1, 0, B)[0]), 5})
    for b in subset:
        # the sequence's pages, gathered into a compact pool (page permutation
        # invariance of the oracle is pinned on the CPU)
        pg = torch.from_numpy(bt[b, :pages[b]].astype(np.int64)).cuda()
        kb = kc[pg].float().cpu().numpy()
        vb = vc[pg].float().cpu().numpy()
        want = ora.verify_attention(q[b * R:(b + 1) * R].float().cpu().numpy(), kb, vb,
                                    np.arange(pages[b], dtype=np.int32)[None], [ctx[b]], [0, R], pos[b * R:(b + 1) * R],
                                    1 / np.sqrt(D), H, Hkv)
        err = assert_close(out[b * R:(b + 1) * R], want, "bf16", f"config4 seq {b} ctx {ctx[b]}")
        print(f"  seq {b} ctx {ctx[b]}: max abs err {err:.2e}", flush=True)


def _load_round(eng, r, prompts, sp):
    """Admit prompts into the round's slots as generate() does (prefill and
    first token included); returns the histories."""
    hists = []
    for b, p in enumerate(prompts):
        s = Sequence(p, sp)
        eng.block_manager.allocate(s)
        eng.block_manager.ensure_capacity(s, len(p) + sp.max_tokens + eng.num_speculative_tokens + 1)
        first = eng._prefill([s])[0]
        h = list(p) + [first]
        hists.append(h)
        r.history[b].zero_()
        r.history[b, :len(h)] = torch.tensor(h, dtype=torch.int32, device="cuda")
        r.hist_len[b] = len(h)
        r.prompt_len[b] = len(p)
        r.max_tokens[b] = sp.max_tokens
        r.max_len[b] = 0
        r.ignore_eos[b] = 1
        r.active[b] = 1
        r.temperature[b] = sp.temperature
        r.block_tables[b].fill_(-1)
        r.block_tables[b, :len(s.block_table)] = torch.tensor(s.block_table, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    return hists


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_config3_round_matches_host_restatement(batch):
    print(f"case: config3 eager round b{batch} vs host restatement (Qwen3-0.6B)", flush=True)
    K = 8
    eng = SpecLLMEngine(dict(spec_method="ngram", num_speculative_tokens=K, ngram_min_size=2, ngram_max_size=4,
                             max_num_sequences=batch, max_model_length=1200 + 16 + 48 + 64, block_size=256,
                             enforce_eager=True, seed=0))
    r = eng.round
    sp = SamplingParams(temperature=0.0, max_tokens=48, ignore_eos=True)
    hists = _load_round(eng, r, synth.config3_prompts(batch), sp)
    r.body(batch)
    torch.cuda.synchronize()
    drafts = [r.drafts[b, :int(r.num_drafts[b])].tolist() for b in range(batch)]
    assert drafts == on.draft(hists, K, 2, 4)
    logits = r.logits[:batch * (K + 1)].float().cpu().numpy()
    accepted = oa.greedy_round(drafts, logits, K + 1)
    for b in range(batch):
        new, _ = orr.commit(hists[b], len(hists[b]) - 1, accepted[b], 48, -1, True, None)
        assert r.history[b, :int(r.hist_len[b])].tolist() == new, b
        assert int(r.committed[b]) == len(accepted[b])
    print(f"  drafted {[len(d) for d in drafts]} accepted {[len(a) for a in accepted]}", flush=True)


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_config3_spec_equals_plain_and_graph_equals_eager(batch):
    print(f"case: config3 b{batch}: 48 greedy tokens, spec == plain, graph == eager (Qwen3-0.6B)", flush=True)
    base = dict(num_speculative_tokens=8, ngram_min_size=2, ngram_max_size=4, max_num_sequences=batch,
                max_model_length=1200 + 16 + 48 + 64, block_size=256, seed=0)
    sp = SamplingParams(temperature=0.0, max_tokens=48, ignore_eos=True)
    prompts = synth.config3_prompts(batch)
    out = {}
    for name, extra in [("spec", {"spec_method": "ngram"}), ("spec_eager", {"spec_method": "ngram",
                                                                            "enforce_eager": True}),
                        ("plain", {"spec_method": "none"})]:
        eng = SpecLLMEngine({**base, **extra})
        res = eng.generate(prompts, sp)
        out[name] = [o["token_ids"] for o in res["outputs"]]
        print(f"  {name}: rounds {res['metrics']['rounds']} {res['metrics']['spec_decoding']}", flush=True)
        del eng
        torch.cuda.empty_cache()
    assert all(len(x) == 48 for x in out["spec"])
    assert out["spec"] == out["spec_eager"]
    assert out["spec"] == out["plain"]


@pytest.mark.parametrize("batch", [1, 8])
def test_config5_stochastic_hybrid_round_matches_oracle(batch):
    print(f"case: config5 stochastic hybrid round b{batch} (0.6B -> 8B, T=1)", flush=True)
    K = 8
    eng = SpecLLMEngine(dict(spec_method="hybrid", num_speculative_tokens=K, ngram_min_size=2, ngram_max_size=4,
                             model_config=Qwen3Config.qwen3_8b(), draft_model_config=Qwen3Config.qwen3_0_6b(),
                             max_num_sequences=batch, max_model_length=1200 + 16 + 48 + 64, block_size=256,
                             enforce_eager=True, seed=5))
    r = eng._round(True)
    sp = SamplingParams(temperature=1.0, max_tokens=48, ignore_eos=True)
    prompts = synth.config3_prompts(batch, seed=5)
    # a random-token question on odd slots, so the batch mixes n-gram and model drafts
    prompts = [p if b % 2 == 0 else p[:1200] + [int(x) for x in synth.randint(b, 94, 6, 100, 151936)]
               for b, p in enumerate(prompts)]
    hists = _load_round(eng, r, prompts, sp)
    r.body(batch)
    torch.cuda.synchronize()
    DL = r.draft_logits[:, :batch].float().cpu().numpy()
    DN = r.draft_noise[:, :batch].cpu().numpy()
    MD = r.model_drafts[:batch].cpu().tolist()
    for b in range(batch):
        for i in range(K):
            assert MD[b][i] == oa.sample(DL[i, b], 1.0, DN[i, b]), (b, i)
    drafts = [r.drafts[b, :int(r.num_drafts[b])].tolist() for b in range(batch)]
    mode = r.draft_mode[:batch].cpu().tolist()
    ng = on.draft(hists, K, 2, 4)
    for b in range(batch):
        assert drafts[b] == (ng[b] if ng[b] else MD[b]) and mode[b] == int(not ng[b]), b
    T = r.logits[:batch * (K + 1)].float().cpu().numpy()
    U = r.uniforms[:batch].cpu().numpy()
    Q = r.accept_noise[:batch].float().cpu().numpy()
    out = r.out_tokens[:batch].cpu().tolist()
    n = r.out_len[:batch].cpu().tolist()
    for b in range(batch):
        k = len(drafts[b])
        rows = T[b * (K + 1): b * (K + 1) + k + 1]
        if mode[b]:
            want = oa.verify(drafts[b], rows, DL[:k, b], 1.0, U[b, :k], Q[b, 0], "bf16")
        else:
            want = oa.verify(drafts[b], rows, None, 1.0, None, Q[b, :k + 1], "bf16")
        assert out[b][:n[b]] == want, (b, out[b][:n[b]], want)
        new, _ = orr.commit(hists[b], len(hists[b]) - 1, want, 48, -1, True, None)
        assert r.history[b, :int(r.hist_len[b])].tolist() == new, b
    print(f"  modes {mode} drafted {[len(d) for d in drafts]} committed {n}", flush=True)
