"""The allocation-free verify-attention entry point
(nsv_verify_attention_noalloc) against the workspace entry point
(nsv_verify_attention), through the C ABI: identical outputs, bit for bit,
on two calls in a row (the second with a smaller input), for each kernel
family that needs scratch: the key-split kernel (split partials and arrival
counters, merged in-kernel), the d-sliced kernel with key splits (partials
merged by a second kernel) and the fp32 kernel with key splits."""

import numpy as np
import pytest
import torch

from naivllm_amd.layers.attention import (paged_attention_verify, verify_attention_plan,
                                          verify_attention_workspace_bytes)
from naivllm_amd.utils import synth
from oracle import attention as ora
from tests.gpu_util import assert_close, to_device

pytestmark = pytest.mark.gpu


def _call(vb, allocation_free):
    t = to_device(vb)
    out = torch.full_like(t["query"], float("nan"))
    paged_attention_verify(t["query"], t["k_cache"], t["v_cache"], t["block_tables"], t["context_lens"],
                           t["cu_seqlens_q"], t["positions"], 1.0 / np.sqrt(vb.head_dim), vb.num_heads,
                           vb.num_kv_heads, vb.head_dim, vb.block_size, 16, max_q_len=vb.max_q_len, out=out,
                           allocation_free=allocation_free)
    torch.cuda.synchronize()
    return out


CASES = {
    # (kernel family, first input, second smaller input)
    "key-split": (dict(ctx=[5000, 3001], q=[9, 9], H=32), dict(ctx=[4100], q=[9], H=32)),
    "d-sliced": (dict(ctx=[1248], q=[9], H=16), dict(ctx=[700], q=[9], H=16)),  # 18 rows: two 16-row tiles
    "fp32": (dict(ctx=[1248, 300], q=[9, 9], H=16, dtype="f32"), dict(ctx=[900], q=[9], H=16, dtype="f32")),
}


@pytest.mark.parametrize("family", list(CASES))
def test_no_alloc_matches_workspace_entry_point(family):
    for i, spec in enumerate(CASES[family]):
        dtype = spec.get("dtype", "bf16")
        vb = synth.verify_batch(40 + i, spec["ctx"], spec["q"], num_heads=spec["H"], num_kv_heads=8, dtype=dtype,
                                max_blocks=24 if family == "key-split" else None)
        tdt = torch.float32 if dtype == "f32" else torch.bfloat16
        kernel, splits = verify_attention_plan(len(spec["ctx"]), spec["H"], 8, 128, 256, vb.block_tables.shape[1],
                                               vb.max_q_len, tdt)
        assert kernel == family and splits > 1, (family, kernel, splits)
        assert verify_attention_workspace_bytes(len(spec["ctx"]), spec["H"], 8, 128, 256, vb.block_tables.shape[1],
                                                vb.max_q_len, tdt) > 0
        print(f"case: no-alloc {family} call {i + 1}: ctx {spec['ctx']} rows {spec['q']} {dtype}, {splits} splits",
              flush=True)
        want = _call(vb, allocation_free=False)
        got = _call(vb, allocation_free=True)
        assert torch.equal(got, want), f"{family} call {i + 1}: allocation-free output differs"
        ref = ora.verify_attention(vb.q, vb.k_cache, vb.v_cache, vb.block_tables, vb.context_lens, vb.cu_seqlens_q,
                                   vb.positions, 1.0 / np.sqrt(vb.head_dim), vb.num_heads, vb.num_kv_heads)
        assert_close(got, ref, dtype, f"{family} call {i + 1} vs oracle")


def test_no_alloc_needs_out():
    vb = synth.verify_batch(1, [300], [9])
    t = to_device(vb)
    with pytest.raises(ValueError, match="preallocated out"):
        paged_attention_verify(t["query"], t["k_cache"], t["v_cache"], t["block_tables"], t["context_lens"],
                               t["cu_seqlens_q"], t["positions"], 0.1, 16, 8, 128, 256, 16, max_q_len=9,
                               allocation_free=True)
