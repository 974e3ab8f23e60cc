"""The drop-in Attention layer driven the way the reference's model layers
drive it (layers/attention.py:689-767): the runner publishes the step's
metadata with set_context, the layer stores the step's K/V at the slots and
attends; results against the oracle (KV store, then verify attention) on
the same inputs, for a verify step and a decode step."""

import numpy as np
import pytest
import torch

from naivllm_amd.layers.attention import Attention
from naivllm_amd.utils import synth
from naivllm_amd.utils.context import get_context, reset_context, set_context
from oracle import attention as ora
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu


def _layer(vb):
    layer = Attention(vb.num_heads, vb.head_dim, scale=1.0, num_kv_heads=vb.num_kv_heads, block_size=vb.block_size)
    f = lambda x: torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda().to(torch.bfloat16)  # noqa: E731
    layer.k_cache, layer.v_cache = f(vb.k_cache), f(vb.v_cache)
    return layer, f


def _slots(vb, positions):
    bs = vb.block_size
    out = []
    row = 0
    for b in range(len(vb.context_lens)):
        for _ in range(vb.cu_seqlens_q[b + 1] - vb.cu_seqlens_q[b]):
            p = int(positions[row])
            out.append(-1 if p < 0 else int(vb.block_tables[b, p // bs]) * bs + p % bs)
            row += 1
    return np.array(out, dtype=np.int64)


def _new_kv(vb, seed):
    T = vb.q.shape[0]
    k = synth.round_to(synth.normal(seed, 5, T * vb.num_kv_heads * vb.head_dim), "bf16")
    v = synth.round_to(synth.normal(seed, 6, T * vb.num_kv_heads * vb.head_dim), "bf16")
    return k.reshape(T, vb.num_kv_heads, vb.head_dim), v.reshape(T, vb.num_kv_heads, vb.head_dim)


def test_verify_step_through_set_context():
    print("case: Attention verify step via set_context", flush=True)
    vb = synth.verify_batch(31, [1210, 300, 77], [9, 9, 4], pad_rows=[0, 2, 0])
    layer, f = _layer(vb)
    slots = _slots(vb, vb.positions)
    k, v = _new_kv(vb, 31)
    qlens = np.diff(vb.cu_seqlens_q).tolist()
    set_context(False, cu_seqlens_q=torch.from_numpy(vb.cu_seqlens_q).cuda(),
                slot_mapping=torch.from_numpy(slots).cuda(), context_lens=torch.from_numpy(vb.context_lens).cuda(),
                block_tables=torch.from_numpy(vb.block_tables).cuda(), seqlens_q=qlens, is_verify=True,
                positions=torch.from_numpy(vb.positions).cuda())
    try:
        assert get_context().is_verify
        out = layer(f(vb.q), f(k), f(v))
        torch.cuda.synchronize()
    finally:
        reset_context()
    assert out.shape == (vb.q.shape[0], vb.num_heads * vb.head_dim)
    kc, vc = vb.k_cache.copy(), vb.v_cache.copy()
    ora.store_kvcache(k, v, kc, vc, slots)
    want = ora.verify_attention(vb.q, kc, vc, vb.block_tables, vb.context_lens, vb.cu_seqlens_q, vb.positions,
                                1 / np.sqrt(vb.head_dim), vb.num_heads, vb.num_kv_heads)
    live = vb.positions >= 0
    got = out.view(-1, vb.num_heads, vb.head_dim)
    assert_close(got[torch.from_numpy(live).cuda()], want[live], "bf16", "verify via set_context")
    # the layer wrote the step's K/V into the caches at the slots
    assert torch.equal(layer.k_cache.float().cpu(), torch.from_numpy(kc).float())
    assert torch.equal(layer.v_cache.float().cpu(), torch.from_numpy(vc).float())


def test_decode_step_through_set_context():
    print("case: Attention decode step via set_context", flush=True)
    vb = synth.verify_batch(32, [513, 1, 256, 1000], [1, 1, 1, 1])
    layer, f = _layer(vb)
    slots = _slots(vb, vb.positions)
    k, v = _new_kv(vb, 32)
    set_context(False, slot_mapping=torch.from_numpy(slots).cuda(), context_lens=torch.from_numpy(vb.context_lens).cuda(),
                block_tables=torch.from_numpy(vb.block_tables).cuda())
    try:
        out = layer(f(vb.q), f(k), f(v))
        torch.cuda.synchronize()
    finally:
        reset_context()
    kc, vc = vb.k_cache.copy(), vb.v_cache.copy()
    ora.store_kvcache(k, v, kc, vc, slots)
    want = ora.verify_attention(vb.q, kc, vc, vb.block_tables, vb.context_lens, vb.cu_seqlens_q, vb.positions,
                                1 / np.sqrt(vb.head_dim), vb.num_heads, vb.num_kv_heads)
    assert_close(out.view(-1, vb.num_heads, vb.head_dim), want, "bf16", "decode via set_context")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_step_through_set_context_paged(dtype):
    # the reference's paged prefill (layers/attention.py:741-752): two prompts,
    # the second behind a 2-page cached prefix; the step stores its K/V at the
    # slots, then every new row attends its sequence's keys 0 .. its position
    print(f"case: Attention paged prefill via set_context {dtype}", flush=True)
    lens, cached = [300, 1210], [0, 128]
    vb = synth.verify_batch(33, lens, [n - c for n, c in zip(lens, cached)], block_size=64, dtype=dtype)
    layer, f = _layer(vb)
    if dtype == "f32":
        f = lambda x: torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda()  # noqa: E731
        layer.k_cache, layer.v_cache = f(vb.k_cache), f(vb.v_cache)
    slots = _slots(vb, vb.positions)
    k, v = _new_kv(vb, 33)
    qlens = [n - c for n, c in zip(lens, cached)]
    set_context(True, cu_seqlens_q=torch.from_numpy(vb.cu_seqlens_q).cuda(),
                cu_seqlens_k=torch.tensor([0, lens[0], sum(lens)], dtype=torch.int32, device="cuda"),
                max_seqlen_q=max(qlens), max_seqlen_k=max(lens), slot_mapping=torch.from_numpy(slots).cuda(),
                block_tables=torch.from_numpy(vb.block_tables).cuda(), seqlens_q=qlens, seqlens_k=lens)
    try:
        out = layer(f(vb.q), f(k), f(v))
        torch.cuda.synchronize()
    finally:
        reset_context()
    kc, vc = vb.k_cache.copy(), vb.v_cache.copy()
    ora.store_kvcache(k, v, kc, vc, slots)
    want = ora.verify_attention(vb.q, kc, vc, vb.block_tables, vb.context_lens, vb.cu_seqlens_q, vb.positions,
                                1 / np.sqrt(vb.head_dim), vb.num_heads, vb.num_kv_heads)
    assert_close(out.view(-1, vb.num_heads, vb.head_dim), want, dtype, "paged prefill via set_context")
    assert torch.equal(layer.k_cache.float().cpu(), torch.from_numpy(kc).float())


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_prefill_step_through_set_context_contiguous(dtype):
    # no block tables (no cached prefix): the reference's varlen flash path
    # (layers/attention.py:754) over the step's own contiguous K/V; a
    # 1100-key prompt needs more than one key split and more than one
    # causal block
    print(f"case: Attention varlen prefill via set_context {dtype}", flush=True)
    H, Hkv, D = 16, 8, 128
    lens = [37, 1100, 5]
    T = sum(lens)
    rnd = lambda st, n: synth.round_to(synth.normal(34, st, n), dtype)  # noqa: E731
    q = rnd(1, T * H * D).reshape(T, H, D)
    k = rnd(2, T * Hkv * D).reshape(T, Hkv, D)
    v = rnd(3, T * Hkv * D).reshape(T, Hkv, D)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    f = lambda x: torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).cuda().to(tdt)  # noqa: E731
    layer = Attention(H, D, scale=1.0, num_kv_heads=Hkv, block_size=256)  # no cache allocated
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    set_context(True, cu_seqlens_q=torch.from_numpy(cu).cuda(), cu_seqlens_k=torch.from_numpy(cu).cuda(),
                max_seqlen_q=max(lens), max_seqlen_k=max(lens), seqlens_q=lens, seqlens_k=lens)
    try:
        out = layer(f(q), f(k), f(v))
        torch.cuda.synchronize()
    finally:
        reset_context()
    # oracle: each sequence as its own one-page cache
    want = []
    for i, n in enumerate(lens):
        sl = slice(cu[i], cu[i + 1])
        want.append(ora.verify_attention(q[sl], k[sl][None], v[sl][None], np.zeros((1, 1), np.int32),
                                         np.array([n]), np.array([0, n], np.int32), np.arange(n),
                                         1 / np.sqrt(D), H, Hkv))
    assert_close(out.view(-1, H, D), np.concatenate(want), dtype, "varlen prefill via set_context")
