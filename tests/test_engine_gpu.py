"""The engine-level drop-in surface (src/myvllm/engine/llm_engine.py:84-152,
spec_engine/spec_llm_engine.py:294-312) and the prefill path:

  * the reference's caller sequence of benchmarks/rag_bench.py:176-197
    (construct, pin_prefix, generate_token_ids, read metrics, exit) runs
    unchanged against naivllm_amd on a small random-init model;
  * more requests than round slots are scheduled through the waiting queue
    and produce the tokens an all-at-once run produces;
  * a warm prefix (pinned) is served from the cache on the next request:
    fewer prefill tokens, prefix-cache hits, the same output;
  * the prefill forward's causal blocks: verify attention over the
    block metadata equals the oracle's attention of the whole sequences.
"""

import numpy as np
import pytest
import torch

from naivllm_amd.layers.attention import paged_attention_verify
from naivllm_amd.layers.qwen3 import Qwen3Config, prefill_metadata
from naivllm_amd.sampling_parameters import SamplingParams
from naivllm_amd.spec_engine import SpecLLMEngine
from naivllm_amd.utils import synth
from oracle import attention as ora
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu

TINY = Qwen3Config(vocab_size=2048, hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64,
                   intermediate_size=512, max_position=4096)


def doc_prompts(seed, n, doc_len=300, q_len=6):
    rng = np.random.default_rng(seed)
    spans = [[int(x) for x in rng.integers(0, 2048, 20)] for _ in range(6)]
    doc = [t for i in range(doc_len // 20) for t in spans[(i * 5) % 6]]
    return [doc + [int(x) for x in rng.integers(0, 2048, q_len)] for _ in range(n)]


def config(**kw):
    base = dict(model_config=TINY, spec_method="ngram", num_speculative_tokens=6, ngram_min_size=2,
                ngram_max_size=4, max_num_sequences=4, max_model_length=512, block_size=64, seed=7)
    base.update(kw)
    return base


def test_reference_caller_sequence():
    print("case: rag_bench caller sequence (pin_prefix, generate_token_ids, metrics, exit)", flush=True)
    prompts = doc_prompts(1, 3)
    eng = SpecLLMEngine(config())
    assert eng.pin_prefix(prompts[0]) == 0  # nothing cached yet: nothing to pin
    params = SamplingParams(temperature=0, max_tokens=24, ignore_eos=True)
    out = eng.generate_token_ids(prompts, params)
    m = out["metrics"]
    for key in ("total_s", "ttft_s", "prefill_tokens", "decode_tokens", "output_tokens", "prefix_cache",
                "spec_decoding"):
        assert key in m, key
    assert [len(t) for t in out["token_ids"]] == [24] * 3
    assert m["output_tokens"] == 72 and 0 < m["ttft_s"] <= m["total_s"]
    assert m["decode_tokens"] == 72 - 3  # the first token of each request comes from its prefill
    st = m["spec_decoding"]
    assert st["method"] == "ngram" and st["rounds"] > 0 and st["accepted_tokens"] <= st["drafted_tokens"] + st["rounds"] * 3
    # the 3 prompts share their 300-token document: 4 full 64-token pages of it
    # are computed once and reused by the other two within the same call
    assert m["prefill_tokens"] == len(prompts[0]) + 2 * (len(prompts[0]) - 4 * 64)
    assert m["prefix_cache"]["hits"] == 2 * 4
    assert eng.pin_prefix(prompts[0]) == 4 * 64
    assert eng.block_manager.cache_stats()["pinned_blocks"] == 4
    eng.exit()
    eng.exit()  # idempotent
    with pytest.raises(RuntimeError):
        eng.generate_token_ids(prompts, params)


def test_context_manager_and_token_id_prompts_only():
    with SpecLLMEngine(config()) as eng:
        with pytest.raises(ValueError, match="tokenizer"):
            eng.generate_token_ids(["a string prompt"], SamplingParams(max_tokens=2))
        assert not eng._closed
    assert eng._closed


def test_waiting_queue_matches_all_at_once():
    print("case: 6 requests through 2 slots == 6 slots", flush=True)
    prompts = [p[:150 + 11 * i] for i, p in enumerate(doc_prompts(2, 6))]
    params = [SamplingParams(temperature=0, max_tokens=10 + 3 * i, ignore_eos=True) for i in range(6)]
    outs = {}
    for slots in (2, 6):
        eng = SpecLLMEngine(config(max_num_sequences=slots, seed=11))
        res = eng.generate_token_ids(prompts, params)
        outs[slots] = res["token_ids"]
        print(f"  {slots} slots: rounds {res['metrics']['rounds']} prefill tokens {res['metrics']['prefill_tokens']}",
              flush=True)
        eng.exit()
        del eng
        torch.cuda.empty_cache()
    assert [len(t) for t in outs[2]] == [10 + 3 * i for i in range(6)]
    assert outs[2] == outs[6]


def test_warm_pinned_prefix_is_reused():
    print("case: warm pinned prefix", flush=True)
    prompt = doc_prompts(3, 1, doc_len=400)[0]
    params = SamplingParams(temperature=0, max_tokens=16, ignore_eos=True)
    eng = SpecLLMEngine(config(seed=13))
    cold = eng.generate_token_ids([prompt], params)
    assert cold["metrics"]["prefill_tokens"] == len(prompt)
    assert eng.pin_prefix(prompt) == 6 * 64
    # another request in between does not evict the pinned pages
    eng.generate_token_ids(doc_prompts(4, 2, doc_len=400), params)
    warm = eng.generate_token_ids([prompt], params)
    assert warm["metrics"]["prefill_tokens"] == len(prompt) - 6 * 64
    assert warm["token_ids"] == cold["token_ids"]
    eng.unpin_all()
    assert eng.block_manager.cache_stats()["pinned_blocks"] == 0
    eng.exit()


@pytest.mark.parametrize("prompt_len,max_tokens", [(100, 28), (127, 1)])
def test_output_ending_on_a_page_boundary_is_not_served_from_cache(prompt_len, max_tokens):
    # the request ends exactly on a page boundary (128 = 2 pages of 64), so its
    # last token has no KV; a follow-up prompt that extends it must recompute
    # that page, and its output must equal a fresh engine's
    print(f"case: page-boundary finish, prompt {prompt_len}, max_tokens {max_tokens}", flush=True)
    prompt = doc_prompts(5, 1, doc_len=300)[0][:prompt_len]
    params = SamplingParams(temperature=0, max_tokens=max_tokens, ignore_eos=True)
    eng = SpecLLMEngine(config(seed=17))
    first = eng.generate_token_ids([prompt], params)["token_ids"][0]
    follow = prompt + first + [3, 1, 4, 1, 5, 9, 2, 6, 5, 3]
    follow_params = SamplingParams(temperature=0, max_tokens=12, ignore_eos=True)
    hits0 = eng.block_manager.cache_stats()["hits"]
    warm = eng.generate_token_ids([follow], follow_params)
    assert eng.block_manager.cache_stats()["hits"] - hits0 == 1  # page 0 only
    assert warm["metrics"]["prefill_tokens"] == len(follow) - 64
    eng.exit()
    fresh_eng = SpecLLMEngine(config(seed=17))
    fresh = fresh_eng.generate_token_ids([follow], follow_params)
    fresh_eng.exit()
    assert warm["token_ids"] == fresh["token_ids"]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_blocks_match_whole_sequence_attention(dtype):
    # two sequences: one prefilled from token 0, one whose first 2 pages are a cached prefix
    print(f"case: prefill causal blocks {dtype}", flush=True)
    H, Hkv, D, bs = 16, 8, 128, 64
    lens, starts = [300, 517], [0, 128]
    vb = synth.verify_batch(61, lens, [n - s for n, s in zip(lens, starts)], num_heads=H, num_kv_heads=Hkv,
                            head_dim=D, block_size=bs, dtype=dtype)
    want = ora.verify_attention(vb.q, vb.k_cache, vb.v_cache, vb.block_tables, vb.context_lens, vb.cu_seqlens_q,
                                vb.positions, 1 / np.sqrt(D), H, Hkv)
    tables = [[int(x) for x in vb.block_tables[b] if x >= 0] for b in range(2)]
    toks = [list(range(n)) for n in lens]
    qb = 64 // (H // Hkv)
    ids, pos, slots, bt, ctx, cu, last = prefill_metadata(toks, starts, tables, bs, qb, "cuda")
    assert pos.tolist() == vb.positions.tolist() and last.tolist() == [lens[0] - 1, sum(lens) - starts[1] - 1]
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    f = lambda x: torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda().to(dt)  # noqa: E731
    out = paged_attention_verify(f(vb.q), f(vb.k_cache), f(vb.v_cache), bt, ctx, cu, pos, 1 / np.sqrt(D), H, Hkv, D,
                                 bs, qb, max_q_len=qb)
    torch.cuda.synchronize()
    assert_close(out, want, dtype, "prefill blocks")
