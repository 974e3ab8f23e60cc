"""torch-on-CPU restatement of the verify path, timed as bench.py's
cpu_baseline (TEST INFRASTRUCTURE ONLY — see oracle/__init__.py).

``paged_verify_attention`` follows the reference's own torch path
``paged_attention_prefill`` (src/myvllm/layers/attention.py:328-363):
gather the sequence's keys through the block table, repeat_interleave the
KV heads, scores in fp32, causal mask from absolute positions, softmax in
fp32, probabilities cast back to the V dtype, einsum with V.  ``greedy_accept``
is the batched argmax + exact-match walk of
src/myvllm/spec_engine/spec_llm_engine.py:224-227 and
rejection_sampler.py:25-36.
"""

from __future__ import annotations

import torch


def paged_verify_attention(q, k_cache, v_cache, block_tables, context_lens, cu_seqlens_q, positions, scale,
                           num_heads, num_kv_heads):
    bs = k_cache.shape[1]
    G = num_heads // num_kv_heads
    out = torch.zeros_like(q)
    for b in range(block_tables.shape[0]):
        L = int(context_lens[b])
        r0, r1 = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        n = torch.arange(L)
        pages = block_tables[b, n // bs].long()
        k = k_cache[pages, n % bs].repeat_interleave(G, dim=1)
        v = v_cache[pages, n % bs].repeat_interleave(G, dim=1)
        qs = q[r0:r1]
        scores = torch.einsum("qhd,khd->hqk", qs, k).float() * scale
        causal = n.unsqueeze(0) <= positions[r0:r1].unsqueeze(1)
        scores.masked_fill_(~causal.unsqueeze(0), torch.finfo(scores.dtype).min)
        p = torch.softmax(scores, dim=-1).to(v.dtype)
        out[r0:r1] = torch.einsum("hqk,khd->qhd", p, v)
    return out


def greedy_accept(draft_tokens: list[list[int]], target_logits: torch.Tensor, stride: int) -> list[list[int]]:
    argmax = target_logits.argmax(dim=-1).tolist()
    result = []
    for i, drafts in enumerate(draft_tokens):
        tgt = argmax[i * stride: i * stride + len(drafts) + 1]
        acc = []
        for d, t in zip(drafts, tgt):
            if d != t:
                acc.append(t)
                break
            acc.append(d)
        else:
            acc.append(tgt[len(drafts)])
        result.append(acc)
    return result
