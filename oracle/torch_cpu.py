"""torch-executed restatements of the reference's torch call sequences —
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

These run the reference's own sequence of torch calls (torch's softmax,
argmax, multinomial and dtype promotion), an arithmetic path independent of
the float64 numpy oracle in oracle/attention.py and oracle/accept.py.  They
serve two roles: bench.py's cpu_baseline times ``paged_verify_attention`` +
``greedy_accept`` on the host's cores, and the tests use
``verify_stochastic`` / ``sample`` as a second, torch-executed check of the
acceptance oracle.

  * ``paged_verify_attention`` — the reference's torch path
    ``paged_attention_prefill`` (src/myvllm/layers/attention.py:328-363):
    gather the sequence's keys through the block table, repeat_interleave
    the KV heads, scores in fp32, causal mask from absolute positions,
    softmax in fp32, probabilities cast back to the V dtype, einsum with V.
  * ``greedy_accept`` — the engine's batched argmax over the padded row
    stride (src/myvllm/spec_engine/spec_llm_engine.py:216-227) and the
    exact-match walk of rejection_sampler.py:25-36.
  * ``verify_stochastic`` — rejection_sampler.py:38-85 with the caller's
    generator (rand(K), then one multinomial per sequence).
  * ``sample`` — SamplerLayer, layers/sampler.py:14-24.

Parity pins (tests/test_oracle_torch_cpu.py): ``paged_verify_attention``
against oracle.attention.verify_attention (itself pinned by torch SDPA, a
brute-force golden fixture and invariances) at 1e-5 in fp32 and 2e-2 abs /
1e-2 rel in bf16, plus the page-permutation invariance; ``greedy_accept``
against oracle.accept.greedy_round on tie-heavy rows and closed forms
(all drafts matching, first draft wrong, empty drafts); ``verify_stochastic``
and ``sample`` against closed forms (identical target and draft rows accept
every draft whose uniform is < 1; a draft the target gives probability 0 is
always rejected and never resampled; greedy rows return the argmax; flat
logits sample argmin of the exponential noise) and decision-for-decision
against oracle.accept on shared random draws.
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
    """Accepted tokens per sequence: one batched argmax over every row, then
    per sequence i (rows i*stride ..) the drafts while they equal the argmax,
    the argmax at the first mismatch, or the bonus argmax after K_i matches."""
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


def verify_stochastic(draft_tokens, target_rows, draft_rows, temperature, g):
    """The reference's stochastic acceptance (rejection_sampler.py:38-85),
    executed by torch on the device of its inputs with generator g."""
    p_target = torch.softmax(target_rows / temperature, dim=-1)
    K = len(draft_tokens)
    acc = []
    if draft_rows is not None:
        p_draft = torch.softmax(draft_rows / temperature, dim=-1)
        ids = torch.tensor(draft_tokens, device=target_rows.device, dtype=torch.long)
        pd = p_draft.gather(1, ids[:, None]).squeeze(1)
        pt = p_target[:-1].gather(1, ids[:, None]).squeeze(1)
        ratio = (pt / pd.clamp_min(1e-20)).clamp(max=1.0)
        u = torch.rand(K, device=target_rows.device, generator=g)
        for i in range(K):
            if u[i] < ratio[i]:
                acc.append(draft_tokens[i])
                continue
            r = (p_target[i] - p_draft[i]).clamp_min(0)
            if r.sum() <= 0:
                r = p_target[i]
            acc.append(int(torch.multinomial(r / r.sum(), 1, generator=g).item()))
            return acc
        acc.append(int(torch.multinomial(p_target[K], 1, generator=g).item()))
        return acc
    s = torch.multinomial(p_target, 1, generator=g).squeeze(1).tolist()
    for i in range(K):
        if s[i] != draft_tokens[i]:
            return acc + [s[i]]
        acc.append(draft_tokens[i])
    return acc + [s[K]]


def sample(logits, temperature, noise):
    """SamplerLayer (layers/sampler.py:14-24): argmax for temperature
    <= 1e-6, else argmax(softmax(logits / T) / noise) with noise ~ Exp(1)."""
    greedy = temperature <= 1e-6
    safe_temperature = torch.where(greedy, torch.ones_like(temperature), temperature)
    argmax_tokens = logits.argmax(dim=-1)
    probs = torch.softmax(logits / safe_temperature.unsqueeze(-1), dim=-1)
    sample_tokens = (probs / noise).argmax(dim=-1)
    return torch.where(greedy, argmax_tokens, sample_tokens)
