"""The model and hybrid drafters inside the device round: the draft-step
metadata kernel against the oracle, the drafts against the draft model's own
greedy decoding, greedy speculative output against plain greedy decoding
(model and hybrid drafts, graph and eager), one stochastic round against a
host restatement of the sampler, the acceptance and the commit on the
round's own logits and random draws, and a drafter identical to the target
being accepted."""

import numpy as np
import pytest
import torch

from naivllm_amd.engine.sequence import Sequence
from naivllm_amd.engine.verify_round import prepare_draft
from naivllm_amd.layers.qwen3 import Qwen3Config
from naivllm_amd.sampling_parameters import SamplingParams
from naivllm_amd.spec_engine.spec_llm_engine import SpecLLMEngine
from naivllm_amd.utils import synth
from oracle import accept as oa
from oracle import ngram as on
from oracle import round as orr

pytestmark = pytest.mark.gpu

TARGET = Qwen3Config(vocab_size=2048, hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64,
                     intermediate_size=512, max_position=4096)
DRAFT = Qwen3Config(vocab_size=2048, hidden_size=128, num_layers=2, num_heads=2, num_kv_heads=1, head_dim=64,
                    intermediate_size=256, max_position=4096)


def i32(x):
    return torch.tensor(x, dtype=torch.int32, device="cuda")


def prompts_with_spans(seed, n, vocab=2048):
    rng = np.random.default_rng(seed)
    out = []
    for b in range(n):
        spans = [[int(x) for x in rng.integers(0, vocab, 10)] for _ in range(4)]
        out.append([t for i in range(8 + b) for t in spans[i % 4]] + spans[1][:3])
    return out


def test_prepare_draft_kernel_matches_oracle():
    print("case: prepare_draft kernel", flush=True)
    B, K, S, bs, MB = 5, 4, 64, 8, 8
    hists = [[int(x) for x in synth.randint(b, 90, L, 0, 50)] for b, L in enumerate([10, 1, 31, 0, 17])]
    active = [1, 1, 1, 1, 0]
    tables = [[int(x) for x in synth.randperm(b, 91, 64)[:MB]] for b in range(B)]
    tables[2][3] = -1
    H = torch.zeros(B, S, dtype=torch.int32)
    for b, h in enumerate(hists):
        H[b, :len(h)] = torch.tensor(h, dtype=torch.int32)
    H = H.cuda()
    i64 = dict(dtype=torch.int64, device="cuda")
    ids0, pos0, slot0 = torch.empty(2 * B, **i64), torch.empty(2 * B, **i64), torch.empty(2 * B, **i64)
    pos, slots, ctx = torch.empty(K * B, **i64), torch.empty(K * B, **i64), torch.empty(K * B, **i64)
    prepare_draft(H, i32([len(h) for h in hists]), i32(tables), bs, i32(active), K, ids0, pos0, slot0, pos, slots,
                  ctx)
    w_ids0, w_pos0, w_slot0, w_pos, w_slots, w_ctx = orr.draft_rows(hists, tables, bs, K, active)
    assert (ids0.tolist(), pos0.tolist(), slot0.tolist()) == (w_ids0, w_pos0, w_slot0)
    flat = lambda m: [x for row in m for x in row]
    assert (pos.tolist(), slots.tolist(), ctx.tolist()) == (flat(w_pos), flat(w_slots), flat(w_ctx))


def _load(eng, r, hists, max_tokens=100, temps=None):
    """Admit histories into round slots (prefill included), as generate does."""
    for b, h in enumerate(hists):
        s = Sequence(h, SamplingParams(temperature=temps[b] if temps else 0.0))
        eng.block_manager.allocate(s)
        eng.block_manager.ensure_capacity(s, len(h) + 64)
        eng._prefill([s])
        r.history[b].zero_()
        r.history[b, :len(h)] = torch.tensor(h, dtype=torch.int32, device="cuda")
        r.hist_len[b] = len(h)
        r.prompt_len[b] = len(h) - 2
        r.max_tokens[b] = max_tokens
        r.max_len[b] = 0
        r.ignore_eos[b] = 1
        r.active[b] = 1
        r.temperature[b] = temps[b] if temps else 0.0
        r.block_tables[b].fill_(-1)
        r.block_tables[b, :len(s.block_table)] = torch.tensor(s.block_table, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()


def test_model_drafts_equal_the_drafters_greedy_decoding():
    # one eager greedy round: the K drafts of each sequence are the draft model's own greedy continuation
    print("case: model drafts == drafter greedy decode", flush=True)
    K = 5
    hists = [h[:40 + 3 * i] for i, h in enumerate(prompts_with_spans(4, 3))]
    eng = SpecLLMEngine(dict(model_config=TARGET, draft_model_config=DRAFT, spec_method="model",
                             num_speculative_tokens=K, max_num_sequences=4, max_model_length=256, block_size=16,
                             enforce_eager=True, seed=5))
    r = eng.round
    _load(eng, r, hists)
    r.body(len(hists))
    torch.cuda.synchronize()
    drafts = [r.drafts[b, :int(r.num_drafts[b])].tolist() for b in range(len(hists))]
    assert [int(x) for x in r.num_drafts[:len(hists)]] == [K] * len(hists)
    dm = eng.draft_model
    # a plain engine whose model has the drafter's shape and seed (the engine seeds its drafter with seed + 1)
    solo = SpecLLMEngine(dict(model_config=DRAFT, spec_method="none", max_num_sequences=4, max_model_length=256,
                              block_size=16, enforce_eager=True, seed=5 + 1))
    for a, b in zip(dm.layers, solo.model.layers):
        assert torch.equal(a["qkv"], b["qkv"]) and torch.equal(a["down"], b["down"])
    del eng
    res = solo.generate(hists, SamplingParams(temperature=0.0, max_tokens=K, ignore_eos=True))
    assert [o["token_ids"] for o in res["outputs"]] == drafts


@pytest.mark.parametrize("method", ["model", "hybrid"])
def test_greedy_spec_equals_plain_decode(method):
    print(f"case: greedy {method} spec == plain, graph == eager", flush=True)
    prompts = prompts_with_spans(7, 3)
    sp = SamplingParams(temperature=0.0, max_tokens=30, ignore_eos=True)
    base = dict(model_config=TARGET, draft_model_config=DRAFT, num_speculative_tokens=4, ngram_min_size=2,
                ngram_max_size=4, max_num_sequences=4, max_model_length=512, block_size=16, seed=3)
    out = {}
    for name, extra in [("spec", {"spec_method": method}), ("spec_eager", {"spec_method": method,
                                                                           "enforce_eager": True}),
                        ("plain", {"spec_method": "none"})]:
        eng = SpecLLMEngine({**base, **extra})
        res = eng.generate(prompts, sp)
        out[name] = [o["token_ids"] for o in res["outputs"]]
        print(name, res["metrics"]["rounds"], res["metrics"]["spec_decoding"], flush=True)
        if name == "spec" and method == "hybrid":
            st = res["metrics"]["spec_decoding"]
            assert st["model_fallback_rounds"] >= 0 and "model_fallback_seqs" in st
        del eng
        torch.cuda.empty_cache()
    assert all(len(x) == 30 for x in out["spec"])
    assert out["spec"] == out["spec_eager"]
    assert out["spec"] == out["plain"]


@pytest.mark.parametrize("method", ["model", "hybrid"])
def test_stochastic_round_matches_host_restatement(method):
    # one eager stochastic round: every draft is the sampler's token on that step's logits and noise,
    # the acceptance is the reference's on the round's logits, uniforms and noise, then _commit
    print(f"case: stochastic {method} round vs host restatement", flush=True)
    K, V = 4, TARGET.vocab_size
    eng = SpecLLMEngine(dict(model_config=TARGET, draft_model_config=DRAFT, spec_method=method,
                             num_speculative_tokens=K, ngram_min_size=2, ngram_max_size=4, max_num_sequences=4,
                             max_model_length=256, block_size=16, enforce_eager=True, seed=9))
    r = eng._round(True)
    prompts = prompts_with_spans(8, 4)
    hists = [prompts[0][:45], prompts[1][:37], [int(x) for x in synth.randint(5, 92, 33, 0, V)], prompts[3][:52]]
    temps = [1.0, 0.7, 1.0, 0.0]
    _load(eng, r, hists, temps=temps)
    B = len(hists)
    r.body(B)
    torch.cuda.synchronize()
    DL = r.draft_logits.float().cpu().numpy()
    DN = r.draft_noise.cpu().numpy()
    MD = r.model_drafts[:B].cpu().tolist()
    for b in range(B):
        for i in range(K):
            assert MD[b][i] == oa.sample(DL[i, b], temps[b], DN[i, b]), (b, i)
    drafts = [r.drafts[b, :int(r.num_drafts[b])].tolist() for b in range(B)]
    mode = r.draft_mode[:B].cpu().tolist()
    if method == "hybrid":
        ng = on.draft(hists, K, 2, 4)
        for b in range(B):
            assert drafts[b] == (ng[b] if ng[b] else MD[b]) and mode[b] == int(not ng[b])
        assert 0 < sum(mode) < B  # the case mixes n-gram and model sequences
    else:
        assert drafts == MD and mode == [1] * B
    T = r.logits[:B * (K + 1)].float().cpu().numpy()
    U = r.uniforms.cpu().numpy()
    Q = r.accept_noise.float().cpu().numpy()
    out = r.out_tokens[:B].cpu().tolist()
    n = r.out_len[:B].cpu().tolist()
    for b in range(B):
        k = len(drafts[b])
        rows = T[b * (K + 1): b * (K + 1) + k + 1]
        if mode[b]:
            noise = Q[b] if method == "model" else Q[b, 0]
            want = oa.verify(drafts[b], rows, DL[:k, b], temps[b], U[b, :k], noise, "bf16")
        else:
            want = oa.verify(drafts[b], rows, None, temps[b], None, Q[b, :k + 1], "bf16")
        assert out[b][:n[b]] == want, (b, out[b][:n[b]], want)
        new, _ = orr.commit(hists[b], len(hists[b]) - 2, want, 100, -1, True, None)
        assert r.history[b, :int(r.hist_len[b])].tolist() == new


def test_identical_drafter_is_accepted():
    # drafter == target (same shape and weights): p_t and p_d agree up to the rounding of two
    # forward shapes, so min(1, p_t/p_d) is ~1 and nearly every draft is accepted at T = 1
    print("case: identical drafter", flush=True)
    K = 4
    eng = SpecLLMEngine(dict(model_config=TARGET, draft_model_config=TARGET, draft_seed=11, spec_method="model",
                             num_speculative_tokens=K, max_num_sequences=4, max_model_length=512, block_size=16,
                             seed=11))
    res = eng.generate(prompts_with_spans(9, 4), SamplingParams(temperature=1.0, max_tokens=40, ignore_eos=True))
    st = res["metrics"]["spec_decoding"]
    print(st, res["metrics"]["rounds"], flush=True)
    assert all(len(o["token_ids"]) == 40 for o in res["outputs"])
    # committed tokens per drafted token: (K + 1) / K when everything is accepted
    assert st["accepted_tokens"] >= 0.9 * st["drafted_tokens"]


def test_drop_in_model_and_hybrid_drafters():
    # the reference's drafter protocol on host Sequences: ModelDrafter.prefill mirrors the prompt,
    # draft() appends K greedy drafts (== the drafter's own greedy decoding) and returns (K, vocab)
    # rows; HybridDrafter takes the n-gram continuation where there is one and the model elsewhere
    print("case: drop-in ModelDrafter / HybridDrafter", flush=True)
    from naivllm_amd.engine.block_manager import BlockManager
    from naivllm_amd.layers.qwen3 import Qwen3Verify
    from naivllm_amd.spec_engine import DraftRunner, HybridDrafter, ModelDrafter, NgramDrafter

    K = 4
    dm = Qwen3Verify(DRAFT, "cuda", seed=21)
    runner = DraftRunner(dm, num_blocks=64, block_size=16)
    bm = BlockManager(64, 16, table_attr="draft_block_table", cached_attr="draft_num_cached_tokens")
    drafter = ModelDrafter(runner, bm, num_speculative_tokens=K)
    prompts = [h[:30] for h in prompts_with_spans(12, 2)]
    seqs = [Sequence(list(p)) for p in prompts]
    drafter.prefill(seqs)
    for s in seqs:
        s.append_token(7)  # the first completion token, after the prefill as in the reference
    assert drafter.can_draft(seqs, K)
    tokens, rows = drafter.draft(seqs)
    assert all(len(t) == K for t in tokens) and all(r.shape == (K, DRAFT.vocab_size) for r in rows)
    for s, p, t in zip(seqs, prompts, tokens):
        assert s.token_ids == p + [7] + t and s.draft_tokens == t
    solo = SpecLLMEngine(dict(model_config=DRAFT, spec_method="none", max_num_sequences=4, max_model_length=256,
                              block_size=16, enforce_eager=True, seed=21))
    res = solo.generate([p + [7] for p in prompts], SamplingParams(temperature=0.0, max_tokens=K, ignore_eos=True))
    assert [o["token_ids"] for o in res["outputs"]] == tokens
    # each row is the drafter's distribution at that step: its argmax is the greedy draft
    assert [r.float().argmax(-1).tolist() for r in rows] == tokens

    # hybrid: sequence 0 repeats its spans (n-gram hit), sequence 1 is random (model fallback)
    seqs = [Sequence(prompts_with_spans(13, 1)[0][:45]), Sequence([int(x) for x in synth.randint(3, 93, 30, 0, 2048)])]
    drafter.prefill(seqs)
    for s in seqs:
        # sequence 0: the token that continues its period-40 span pattern
        s.append_token(int(s.token_ids[-40]) if len(s.token_ids) >= 40 else 7)
    hyb = HybridDrafter(NgramDrafter(num_speculative_tokens=K, min_ngram_size=2, max_ngram_size=4), drafter)
    before = [list(s.token_ids) for s in seqs]
    lists, rows = hyb.draft(seqs)
    ng = on.draft(before, K, 2, 4)
    assert ng[0] and not ng[1]
    assert lists[0] == ng[0] and rows[0] is None
    assert len(lists[1]) == K and rows[1] is not None and rows[1].shape == (K, DRAFT.vocab_size)
    assert hyb.model_rounds == 1 and hyb.model_seqs == 1


def test_draft_runner_graphs_match_eager():
    # the graphed K-step draft loop (one graph per batch bucket, replayed from
    # static buffers) against the eager loop on identical weights: identical
    # greedy drafts and logits, for 3 sequences (bucket 4, one inert pad row)
    # over three calls (capture, then two replays with new lengths), then 1
    print("case: DraftRunner graphs == eager", flush=True)
    from naivllm_amd.engine.block_manager import BlockManager
    from naivllm_amd.layers.qwen3 import Qwen3Verify
    from naivllm_amd.spec_engine import DraftRunner

    K = 5
    runs = {}
    for graphed in (True, False):
        dm = Qwen3Verify(DRAFT, "cuda", seed=23)
        runner = DraftRunner(dm, num_blocks=64, block_size=16, use_graphs=graphed)
        bm = BlockManager(64, 16, table_attr="draft_block_table", cached_attr="draft_num_cached_tokens")
        seqs = [Sequence(list(p[:20 + 7 * i])) for i, p in enumerate(prompts_with_spans(14, 3))]
        for s in seqs:
            bm.allocate(s)
            bm.ensure_capacity(s, len(s) + 3 * (K + 1))
        runner.prefill(seqs)
        out = []
        temps = torch.zeros(len(seqs))
        for call in range(3):
            toks, logits = runner.run_draft_steps(seqs, K, temps)
            out.append((toks, logits.float().cpu().clone()))
            for s, t in zip(seqs, toks):  # commit two drafts, as an acceptance would
                s.append_token(t[0])
                s.append_token(t[1])
        toks, logits = runner.run_draft_steps(seqs[:1], K, temps[:1])
        out.append((toks, logits.float().cpu().clone()))
        runs[graphed] = out
        assert (len(runner._graphs) == 2) == graphed  # buckets 4 and 1
    for (tg, lg), (te, le) in zip(runs[True], runs[False]):
        assert tg == te
        assert torch.equal(lg, le)
