"""CPU oracle of the acceptance step — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker; the product path never calls it.

Restates, in float64 numpy with the reference's dtype flow made explicit:
  * greedy acceptance — src/myvllm/spec_engine/rejection_sampler.py:25-36,
    fed by the batched argmax of spec_llm_engine.py:224-227 and the padded
    row stride of :216-219, :229-243;
  * stochastic acceptance — rejection_sampler.py:38-85 and the temperature
    dispatch of :87-98;
  * token sampling of the decode / draft forward — layers/sampler.py:14-24
    (SamplerLayer: argmax, or argmax(softmax(logits / T) / q) in fp32).

Randomness is an input.  The reference draws ``torch.rand(K)`` and then one
``torch.multinomial`` per sequence; torch implements multinomial(p, 1) as
argmax(p / q) with q = empty_like(p).exponential_(1) drawn from the same
generator (checked against torch in tests/test_oracle_accept.py), so the
oracle takes the uniforms ``u`` (float32) and the exponential noise ``q``
(in the probabilities' dtype) and reproduces every decision from them.

Arithmetic model (what "bit-exact" means here).  Every torch op on bf16 or
fp32 tensors computes in fp32 and rounds its result to the tensor dtype:
  * x / T, p_t / p_d, residual / sum, p / q: fp32 IEEE division, then
    rounded to the dtype (``div_round``);
  * p_t - p_d: fp32 subtraction, rounded;
  * softmax and sum: defined here as the exact value (float64 arithmetic)
    rounded to fp32 and then to the dtype.  torch accumulates them in fp32
    in an implementation-defined order; the two agree except when the exact
    value lies within the fp32 accumulation error of a rounding boundary
    (measured in tests/test_oracle_accept.py).
  * argmax: first index of the maximum; NaN counts as the maximum (torch).
"""

from __future__ import annotations

import numpy as np

DTYPES = ("f32", "bf16")


def round_to(x, dtype: str) -> np.ndarray:
    """Round to float32, then (bf16) to bfloat16 with round-to-nearest-even;
    returned as float64 holding exactly representable values."""
    f = np.asarray(x, dtype=np.float64).astype(np.float32)
    if dtype == "f32":
        return f.astype(np.float64)
    if dtype != "bf16":
        raise ValueError(dtype)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) & np.uint64(0xFFFF0000)
    out = u.astype(np.uint32).view(np.float32).astype(np.float64)
    return np.where(nan, np.nan, out)


def div_round(a, b, dtype: str) -> np.ndarray:
    """torch's a / b on dtype tensors: fp32 division, rounded to dtype."""
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.asarray(a, dtype=np.float32) / np.asarray(b, dtype=np.float32)
    return round_to(q, dtype)


def argmax_first(v) -> int:
    """torch.argmax over one row: NaN wins (first NaN), else the first
    index of the maximum."""
    v = np.asarray(v, dtype=np.float64)
    nan = np.isnan(v)
    if nan.any():
        return int(np.argmax(nan))
    return int(np.argmax(v))  # numpy also returns the first maximum


def softmax_rows(x, temperature: float, dtype: str) -> np.ndarray:
    """torch.softmax(x / temperature, dim=-1) for x of ``dtype``
    (rejection_sampler.py:47, :52): the exact softmax of the rounded
    quotient, rounded to the dtype."""
    z = div_round(np.atleast_2d(x), np.float32(temperature), dtype)
    m = z.max(axis=-1, keepdims=True)
    e = np.exp(z - m)
    return round_to(e / e.sum(axis=-1, keepdims=True), dtype)


def sum_round(x, dtype: str) -> float:
    """torch's .sum() of a dtype tensor: exact sum rounded to fp32, then to
    the dtype."""
    return float(round_to(np.sum(np.asarray(x, dtype=np.float64)), dtype))


def multinomial(p, q, dtype: str) -> int:
    """torch.multinomial(p, 1) given its exponential noise q."""
    return argmax_first(div_round(p, q, dtype))


def verify_greedy(draft_tokens, target_tokens) -> list[int]:
    """rejection_sampler.py:25-36 on ready argmax tokens: accept drafts while
    they equal the target's argmax, emit the first disagreeing argmax, or
    the bonus argmax when every draft was accepted."""
    accepted = []
    for d, t in zip(draft_tokens, target_tokens):
        if d != t:
            return accepted + [int(t)]
        accepted.append(int(d))
    accepted.append(int(target_tokens[len(draft_tokens)]))
    return accepted


def greedy_round(draft_lists, target_logits, stride: int | None = None) -> list[list[int]]:
    """The engine's all-greedy round (spec_llm_engine.py:224-243): one
    argmax over every row of target_logits [rows, V], then per sequence the
    rows start at i*stride (graphed, padded to K+1) or packed back to back
    (stride None)."""
    logits = np.asarray(target_logits, dtype=np.float64)
    tokens = [argmax_first(r) for r in logits]
    out, row = [], 0
    for drafts in draft_lists:
        k = len(drafts)
        out.append(verify_greedy(drafts, tokens[row:row + k + 1]))
        row += stride if stride is not None else k + 1
    return out


def verify_stochastic(draft_tokens, target_rows, draft_rows, temperature: float, uniforms, noise,
                      dtype: str) -> list[int]:
    """rejection_sampler.py:38-85 with injected randomness.

    target_rows [K+1, V] and draft_rows [K, V] (or None) hold values of
    ``dtype``; uniforms [K] float32; noise: [V] (draft rows given: the one
    multinomial of the resample or the bonus) or [K+1, V] (no draft rows:
    the row-wise target samples), in ``dtype``.
    """
    K = len(draft_tokens)
    p_t = softmax_rows(target_rows, temperature, dtype)
    accepted: list[int] = []
    if draft_rows is not None:
        p_d = softmax_rows(draft_rows, temperature, dtype)
        floor = float(round_to(1e-20, dtype))
        u = np.asarray(uniforms, dtype=np.float32)
        for i, d in enumerate(draft_tokens):
            pd = max(float(p_d[i, d]), floor)                         # :56 clamp_min(1e-20)
            ratio = min(float(div_round(p_t[i, d], pd, dtype)), 1.0)  # :56 clamp(max=1)
            if float(u[i]) < ratio:                                    # :59 strict <
                accepted.append(int(d))
                continue
            residual = np.maximum(round_to(p_t[i].astype(np.float32) - p_d[i].astype(np.float32), dtype), 0.0)
            if sum_round(residual, dtype) <= 0:                        # :64-65
                residual = p_t[i]
            prob = div_round(residual, sum_round(residual, dtype), dtype)  # :66-67
            accepted.append(multinomial(prob, noise, dtype))
            return accepted
        accepted.append(multinomial(p_t[K], noise, dtype))              # :71-72 bonus
        return accepted
    noise = np.asarray(noise)
    samples = [multinomial(p_t[r], noise[r], dtype) for r in range(K + 1)]  # :76-77
    for i in range(K):
        if samples[i] == draft_tokens[i]:
            accepted.append(int(draft_tokens[i]))
        else:
            accepted.append(samples[i])
            return accepted
    accepted.append(samples[K])
    return accepted


def verify(draft_tokens, target_rows, draft_rows=None, temperature: float = 0.0, uniforms=None, noise=None,
           dtype: str = "f32") -> list[int]:
    """rejection_sampler.py:87-98: greedy when temperature <= 1e-6."""
    if temperature <= 1e-6:
        rows = np.asarray(target_rows, dtype=np.float64)
        return verify_greedy(draft_tokens, [argmax_first(r) for r in rows])
    return verify_stochastic(draft_tokens, target_rows, draft_rows, temperature, uniforms, noise, dtype)


def sample(logits_row, temperature: float, noise_row) -> int:
    """layers/sampler.py:14-24 for one row: temperature <= 1e-6 takes the
    argmax of the logits; otherwise logits / T (a float32 tensor divisor,
    so the quotient, the softmax and probs / noise are float32) and
    argmax(probs / noise) with noise the fp32 exponential draws (already
    clamped at 1e-10 by the caller, :23)."""
    x = np.asarray(logits_row, dtype=np.float64)
    if temperature <= 1e-6:
        return argmax_first(x)
    p = softmax_rows(x, np.float32(temperature), "f32")[0]
    return multinomial(p, np.asarray(noise_row, dtype=np.float32), "f32")


def sample_rows(logits, temperatures, noise) -> list[int]:
    """sample() over the rows of logits [B, V] with temperatures [B] and
    noise [B, V]."""
    return [sample(logits[b], float(temperatures[b]), noise[b]) for b in range(len(temperatures))]
