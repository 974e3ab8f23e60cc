"""Pins the CPU attention oracle (oracle/attention.py) before any GPU result
is compared with it: golden fixture, torch SDPA closed form, invariances."""

import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from naivllm_amd.utils import synth
from oracle import attention as ora

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_tiny.json")


def _run(vb, scale=None):
    scale = scale if scale is not None else 1.0 / np.sqrt(vb.head_dim)
    return ora.verify_attention(vb.q, vb.k_cache, vb.v_cache, vb.block_tables, vb.context_lens,
                                vb.cu_seqlens_q, vb.positions, scale, vb.num_heads, vb.num_kv_heads)


def test_oracle_matches_golden_fixture():
    c = json.load(open(GOLDEN))
    out = ora.verify_attention(np.array(c["q"]), np.array(c["k_cache"]), np.array(c["v_cache"]),
                               np.array(c["block_tables"]), c["context_lens"], c["cu_seqlens_q"],
                               c["positions"], c["scale"], c["num_heads"], c["num_kv_heads"])
    np.testing.assert_allclose(out, np.array(c["expected"]), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("H,Hkv", [(16, 8), (32, 8), (4, 4)])
def test_oracle_matches_sdpa_bottom_right_causal(H, Hkv):
    # torch's own attention on contiguous K/V, with GQA and the bottom-right
    # causal mask a multi-token verify uses (row t of a q_len chunk at the end
    # of an L-token context sees keys 0 .. L - q_len + t)
    vb = synth.verify_batch(5, [37, 70, 9], [9, 4, 9], num_heads=H, num_kv_heads=Hkv, head_dim=16,
                            block_size=8, dtype="f32")
    scale = 0.3
    out = _run(vb, scale)
    bs = vb.block_size
    for b, L in enumerate(vb.context_lens):
        r0, r1 = vb.cu_seqlens_q[b], vb.cu_seqlens_q[b + 1]
        n = np.arange(L)
        pages = vb.block_tables[b, n // bs]
        K = torch.tensor(vb.k_cache[pages, n % bs]).permute(1, 0, 2)[None]   # [1, Hkv, L, D]
        V = torch.tensor(vb.v_cache[pages, n % bs]).permute(1, 0, 2)[None]
        Q = torch.tensor(vb.q[r0:r1]).permute(1, 0, 2)[None]                   # [1, H, q, D]
        ql = r1 - r0
        mask = torch.ones(ql, L, dtype=torch.bool).tril(diagonal=int(L) - ql)
        ref = F.scaled_dot_product_attention(Q, K, V, attn_mask=mask, scale=scale, enable_gqa=True)
        np.testing.assert_allclose(out[r0:r1], ref[0].permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-10)


def test_oracle_invariant_to_page_permutation_and_unmapped_pages():
    vb = synth.verify_batch(6, [40, 23], [9, 5], num_heads=8, num_kv_heads=4, head_dim=8, block_size=8,
                            num_blocks=16, dtype="f32")
    base = _run(vb)
    # move every page to a new physical slot
    perm = synth.randperm(99, 0, 16)
    k2 = np.empty_like(vb.k_cache)
    v2 = np.empty_like(vb.v_cache)
    k2[perm] = vb.k_cache
    v2[perm] = vb.v_cache
    bt2 = np.where(vb.block_tables >= 0, perm[np.maximum(vb.block_tables, 0)], -1).astype(np.int32)
    moved = ora.verify_attention(vb.q, k2, v2, bt2, vb.context_lens, vb.cu_seqlens_q, vb.positions,
                                 1 / np.sqrt(8), 8, 4)
    np.testing.assert_allclose(moved, base, rtol=1e-12, atol=1e-12)
    # garbage in pages no table maps must not matter
    used = set(vb.block_tables[vb.block_tables >= 0].tolist())
    k3, v3 = vb.k_cache.copy(), vb.v_cache.copy()
    for p in range(16):
        if p not in used:
            k3[p] = 1e6
            v3[p] = -1e6
    vb.k_cache, vb.v_cache = k3, v3
    np.testing.assert_allclose(_run(vb), base, rtol=1e-12, atol=1e-12)


def test_every_row_equals_a_decode_at_its_position():
    vb = synth.verify_batch(7, [50], [9], num_heads=4, num_kv_heads=2, head_dim=8, block_size=16, dtype="f32")
    full = _run(vb)
    for r in range(9):
        pos = int(vb.positions[r])
        one = ora.verify_attention(vb.q[r:r + 1], vb.k_cache, vb.v_cache, vb.block_tables,
                                   np.array([pos + 1]), np.array([0, 1]), np.array([pos]),
                                   1 / np.sqrt(8), 4, 2)
        np.testing.assert_allclose(one[0], full[r], rtol=1e-12, atol=1e-12)


def test_pad_rows_and_empty_sequences_are_zero():
    vb = synth.verify_batch(8, [20, 0], [4, 2], num_heads=4, num_kv_heads=2, head_dim=8, block_size=8,
                            dtype="f32", pad_rows=[2, 0])
    out = _run(vb)
    assert np.all(out[2:4] == 0) and np.all(out[4:6] == 0)
    assert np.all(np.abs(out[:2]) > 0)


def test_oracle_store_kvcache_scatter():
    key = np.arange(3 * 2 * 4, dtype=np.float64).reshape(3, 2, 4)
    val = -key
    kc = np.zeros((3, 4, 2, 4))
    vc = np.zeros((3, 4, 2, 4))
    ora.store_kvcache(key, val, kc, vc, [5, -1, 11])
    assert np.array_equal(kc[1, 1], key[0]) and np.array_equal(kc[2, 3], key[2])
    assert np.array_equal(vc[2, 3], -key[2])
    assert np.count_nonzero(kc) == 2 * 2 * 4 - 1  # key[0] holds one zero; slot -1 wrote nothing
