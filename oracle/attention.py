"""CPU oracle for verify attention and the paged KV store.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only as the
checker; the product path (naivllm_amd) never calls it.

Restates the reference's semantics in float64 numpy:
  * verify attention — src/myvllm/layers/attention.py:522-612 (mask and
    padding semantics of the Triton kernel) with the math of the
    reference's own torch restatement ``paged_attention_prefill``
    (:328-363): keys are gathered through the block table
    (physical = block_tables[b, j // bs], offset j % bs, :564-571), GQA
    maps head h to kv head h // (H / Hkv) (:549, and repeat_interleave at
    :349-350), query row r attends keys j <= positions[r] (:595) with
    j < context_lens[b] and a mapped page (:568-569).
  * KV store — :9-68: cache[slot // bs, slot % bs] = row, slot -1 skipped.

Pad rows (position -1) are inert in the reference and never read; the
oracle defines them as zeros, matching the library.

Parity pins (tests/test_oracle_attention.py): torch's
scaled_dot_product_attention on materialised contiguous K/V with the
bottom-right causal mask; a pure-Python brute force and the committed
golden fixture on tiny shapes; invariance to the physical page
permutation and to unmapped pool contents; every row equal to a decode
(one query row) at its own position.
"""

from __future__ import annotations

import numpy as np


def verify_attention(q, k_cache, v_cache, block_tables, context_lens, cu_seqlens_q, positions, scale,
                     num_heads: int, num_kv_heads: int) -> np.ndarray:
    q = np.asarray(q, dtype=np.float64)
    k_cache = np.asarray(k_cache)
    v_cache = np.asarray(v_cache)
    block_tables = np.asarray(block_tables)
    T, H, D = q.shape
    if H != num_heads:
        raise ValueError("query heads disagree with num_heads")
    nb, bs, hkv, _ = k_cache.shape
    if hkv != num_kv_heads or H % hkv:
        raise ValueError("bad kv head count")
    G = H // hkv
    max_ctx = block_tables.shape[1] * bs  # the reference never walks past the table width
    out = np.zeros((T, H, D), dtype=np.float64)
    for b in range(block_tables.shape[0]):
        L = min(int(context_lens[b]), max_ctx)
        r0, r1 = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        if r1 <= r0 or L <= 0:
            continue
        n = np.arange(L)
        page = block_tables[b, n // bs].astype(np.int64)
        mapped = page >= 0
        keys = n[mapped]
        rows = [r for r in range(r0, r1) if int(positions[r]) >= 0]
        if not rows or keys.size == 0:
            continue
        pos = np.array([int(positions[r]) for r in rows])
        visible = keys[None, :] <= pos[:, None]  # [rows, Lk]
        for hk in range(hkv):  # kv head hk serves query heads hk*G .. hk*G+G-1
            K = k_cache[page[mapped], (n % bs)[mapped], hk].astype(np.float64)  # [Lk, D]
            V = v_cache[page[mapped], (n % bs)[mapped], hk].astype(np.float64)
            for g in range(G):
                h = hk * G + g
                s = (q[rows, h] @ K.T) * scale  # [rows, Lk]
                s = np.where(visible, s, -np.inf)
                m = s.max(axis=1, keepdims=True)
                ok = np.isfinite(m[:, 0])  # a row with no visible key keeps zeros
                p = np.exp(s - np.where(np.isfinite(m), m, 0.0))
                p /= np.maximum(p.sum(axis=1, keepdims=True), 1e-300)
                o = p @ V
                for i, r in enumerate(rows):
                    if ok[i]:
                        out[r, h] = o[i]
    return out


def store_kvcache(key, value, k_cache, v_cache, slot_mapping) -> None:
    """In-place scatter of [T, Hkv, D] rows into [nb, bs, Hkv, D] caches."""
    bs = k_cache.shape[1]
    for t, slot in enumerate(np.asarray(slot_mapping)):
        slot = int(slot)
        if slot < 0:
            continue
        k_cache[slot // bs, slot % bs] = key[t]
        v_cache[slot // bs, slot % bs] = value[t]
