"""ModelRunner.run_spec_verify (src/myvllm/engine/model_runner.py:724-777):
host Sequences with appended drafts in, target logits out; graphed rows at
stride K + 1 (inert pad rows), eager rows packed; both equal to the verify
forward called directly on the same rows."""

import pytest
import torch

from naivllm_amd.engine.block_manager import BlockManager
from naivllm_amd.engine.model_runner import ModelRunner
from naivllm_amd.engine.sequence import Sequence
from naivllm_amd.layers.qwen3 import Qwen3Config, Qwen3Verify
from naivllm_amd.utils import synth
from naivllm_amd.utils.context import get_context, reset_context

pytestmark = pytest.mark.gpu

TINY = Qwen3Config(vocab_size=2048, hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64,
                   intermediate_size=512, max_position=4096)
K = 4


def setup(seed):
    model = Qwen3Verify(TINY, "cuda", seed=seed)
    model.allocate_kv_cache(64, 16)
    bm = BlockManager(64, 16)
    seqs = []
    for i, (n, k) in enumerate([(40, 4), (23, 0), (57, 2)]):
        s = Sequence([int(x) for x in synth.randint(seed, 70 + i, n, 0, 2048)])
        bm.allocate(s)
        bm.ensure_capacity(s, n + K + 1)
        model.prefill([s.token_ids], [0], [s.block_table])
        s.append_token(int(synth.randint(seed, 80 + i, 1, 0, 2048)[0]))  # the confirmed token from the prefill
        drafts = [int(x) for x in synth.randint(seed, 90 + i, k, 0, 2048)]
        for d in drafts:
            s.append_token(d)
        s.draft_tokens = drafts
        seqs.append(s)
    torch.cuda.synchronize()
    return model, seqs


def test_graphed_rows_at_stride_k_plus_1():
    print("case: run_spec_verify graphed / eager", flush=True)
    model, seqs = setup(3)
    runner = ModelRunner(model, max_num_sequences=4, num_spec_tokens=K, max_model_length=256)
    assert runner.verify_vars["k"] == K and sorted(runner.verify_graphs) == [1, 2, 4]
    got = runner.run_spec_verify(seqs).clone()
    torch.cuda.synchronize()
    assert got.shape == (4 * (K + 1), TINY.vocab_size)  # bucket 4 for 3 sequences
    # the same padded rows through the forward directly: identical logits
    v = runner.verify_vars
    rows = 4 * (K + 1)
    want = model.forward(v["input_ids"][:rows], v["positions"][:rows], v["slot_mapping"][:rows],
                         v["block_tables"][:4], v["context_lens"][:4],
                         torch.arange(0, rows + 1, K + 1, dtype=torch.int32, device="cuda"), K + 1)
    assert torch.equal(got, want)
    # rows of sequence i start at i * (K + 1) and hold its [last_confirmed, drafts]
    for i, s in enumerate(seqs):
        n = len(s) - len(s.draft_tokens)
        assert v["positions"][i * (K + 1): i * (K + 1) + len(s.draft_tokens) + 1].tolist() == list(range(n - 1, len(s)))
        assert v["positions"][i * (K + 1) + len(s.draft_tokens) + 1: (i + 1) * (K + 1)].tolist() == \
            [-1] * (K - len(s.draft_tokens))
    # eager: packed rows, equal to a direct forward on the packed rows
    eager = ModelRunner(model, max_num_sequences=4, num_spec_tokens=K, max_model_length=256, enforce_eager=True)
    packed = eager.run_spec_verify(seqs)
    assert not get_context().is_verify  # run_spec_verify resets the context after its forward
    # prepare_spec_verify publishes the step's Context (model_runner.py:467-480) and returns the input_ids
    ids = eager.prepare_spec_verify(seqs)
    c = get_context()
    try:
        assert c.is_prefill and c.is_verify and c.cu_seqlens_k is None
        assert c.seqlens_q == [len(s.draft_tokens) + 1 for s in seqs] and c.seqlens_k == [len(s) for s in seqs]
        assert c.max_seqlen_q == max(c.seqlens_q) and c.max_seqlen_k == max(c.seqlens_k)
        assert ids.dtype == torch.int64 and ids.shape[0] == sum(c.seqlens_q)
        assert c.positions.tolist() == [p for s in seqs for p in range(len(s) - len(s.draft_tokens) - 1, len(s))]
        want_packed = model.forward(ids, c.positions, c.slot_mapping, c.block_tables, c.context_lens,
                                    c.cu_seqlens_q, c.max_seqlen_q)
    finally:
        reset_context()
    assert torch.equal(packed, want_packed)
    assert packed.shape[0] == sum(len(s.draft_tokens) + 1 for s in seqs)
    # the two layouts agree row for row (bf16 logits of two batch shapes)
    r = 0
    for i, s in enumerate(seqs):
        m = len(s.draft_tokens) + 1
        torch.testing.assert_close(packed[r:r + m].float(), got[i * (K + 1): i * (K + 1) + m].float(),
                                   atol=5e-2, rtol=2e-2)
        r += m


def test_rejects_oversized_batches_and_drafts():
    model, seqs = setup(5)
    runner = ModelRunner(model, max_num_sequences=2, num_spec_tokens=K, max_model_length=256)
    with pytest.raises(ValueError):
        runner.run_spec_verify(seqs)  # 3 sequences, 2 slots
    s = seqs[0]
    s.draft_tokens = s.draft_tokens + [1]  # K + 1 drafts
    with pytest.raises(ValueError):
        runner.run_spec_verify([s])
