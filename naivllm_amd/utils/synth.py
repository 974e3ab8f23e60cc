"""Seeded synthetic inputs for the verify round.

A self-contained counter-based generator (splitmix64 finalizer over
``seed``/``stream``/index, Box-Muller for normals) so that the same seed
produces bit-identical inputs on any host, independent of a library's RNG
stream.  Used by bench.py and the tests; results never depend on torch's
or numpy's generators.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def random_bits(seed: int, stream: int, n: int) -> np.ndarray:
    """n pseudo-random uint64 values for (seed, stream)."""
    with np.errstate(over="ignore"):
        key = _mix(np.array([seed & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64) * _GOLDEN
                   + np.uint64(stream & 0xFFFFFFFF))
        idx = np.arange(1, n + 1, dtype=np.uint64)
        return _mix(key + idx * _GOLDEN)


def uniform(seed: int, stream: int, n: int) -> np.ndarray:
    """float64 uniforms in [0, 1)."""
    return (random_bits(seed, stream, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, stream: int, n: int, std: float = 1.0) -> np.ndarray:
    """float64 N(0, std^2) samples (Box-Muller on pairs of uniforms)."""
    m = (n + 1) // 2
    u = uniform(seed, stream, 2 * m)
    r = np.sqrt(-2.0 * np.log1p(-u[:m]))  # 1 - u in (0, 1]
    th = 2.0 * math.pi * u[m:]
    z = np.empty(2 * m)
    z[0::2] = r * np.cos(th)
    z[1::2] = r * np.sin(th)
    return z[:n] * std


def randint(seed: int, stream: int, n: int, low: int, high: int) -> np.ndarray:
    """int64 values uniform in [low, high)."""
    span = np.uint64(high - low)
    return (random_bits(seed, stream, n) % span).astype(np.int64) + low


def randperm(seed: int, stream: int, n: int) -> np.ndarray:
    return np.argsort(random_bits(seed, stream, n), kind="stable").astype(np.int64)


@dataclass
class VerifyBatch:
    """Inputs of one verify-attention call, as numpy arrays (float64 values
    already rounded to ``dtype``'s precision)."""
    q: np.ndarray             # [T, H, D]
    k_cache: np.ndarray       # [num_blocks, block_size, Hkv, D]
    v_cache: np.ndarray
    block_tables: np.ndarray  # [B, max_blocks] int32, -1 padded
    context_lens: np.ndarray  # [B] int64
    cu_seqlens_q: np.ndarray  # [B+1] int32
    positions: np.ndarray     # [T] int64, -1 = inert pad row
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: str                # "f32" | "bf16"

    @property
    def max_q_len(self) -> int:
        return int(np.max(np.diff(self.cu_seqlens_q))) if len(self.cu_seqlens_q) > 1 else 1


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float64 values to float32 or bfloat16 (round-to-nearest-even),
    returned as float64 holding exactly representable values."""
    f = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return f.astype(np.float64)
    if dtype != "bf16":
        raise ValueError(dtype)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) & np.uint64(0xFFFF0000)
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def verify_batch(seed: int, ctx_lens, q_lens, *, num_heads: int = 16, num_kv_heads: int = 8,
                 head_dim: int = 128, block_size: int = 256, num_blocks: int | None = None,
                 max_blocks: int | None = None, dtype: str = "bf16", pad_rows=None) -> VerifyBatch:
    """A verify batch over a shared page pool.

    Sequence b has context ctx_lens[b] (its drafts included) and q_lens[b]
    query rows at positions ctx-q_len .. ctx-1.  Its pages are taken from one
    seeded permutation of the pool, so pages are disjoint across sequences
    and scattered over the pool; the whole pool (mapped or not) is filled
    with N(0,1).  ``pad_rows``: optional per-sequence count of trailing rows
    replaced by inert padding (position -1), as the reference's graphed
    verify pads rows to K+1.
    """
    ctx_lens = [int(x) for x in ctx_lens]
    q_lens = [int(x) for x in q_lens]
    B = len(ctx_lens)
    pages = [(c + block_size - 1) // block_size for c in ctx_lens]
    need = sum(pages)
    if num_blocks is None:
        num_blocks = max(need, 1) + 4
    if need > num_blocks:
        raise ValueError("pool too small")
    if max_blocks is None:
        max_blocks = max(max(pages) if pages else 1, 1)
    perm = randperm(seed, 1, num_blocks)
    bt = np.full((B, max_blocks), -1, dtype=np.int32)
    off = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    T = sum(q_lens)
    H, Hkv, D = num_heads, num_kv_heads, head_dim
    q = round_to(normal(seed, 2, T * H * D), dtype).reshape(T, H, D)
    pool = num_blocks * block_size * Hkv * D
    k = round_to(normal(seed, 3, pool), dtype).reshape(num_blocks, block_size, Hkv, D)
    v = round_to(normal(seed, 4, pool), dtype).reshape(num_blocks, block_size, Hkv, D)
    cu = np.zeros(B + 1, dtype=np.int32)
    cu[1:] = np.cumsum(q_lens)
    pos = np.empty(T, dtype=np.int64)
    for b in range(B):
        pos[cu[b]:cu[b + 1]] = np.arange(ctx_lens[b] - q_lens[b], ctx_lens[b])
        if pad_rows is not None and pad_rows[b]:
            pos[cu[b + 1] - pad_rows[b]:cu[b + 1]] = -1
    return VerifyBatch(q, k, v, bt, np.asarray(ctx_lens, dtype=np.int64), cu, pos, H, Hkv, D, block_size, dtype)


def config1_batch(seed: int = 1) -> VerifyBatch:
    """b1 fp32, L=1248, 5 pages of a 64-page pool, K=8."""
    return verify_batch(seed, [1248], [9], num_blocks=64, dtype="f32")


def config2_ctx_lens(seed: int = 2, batch: int = 8) -> list[int]:
    """BASELINE config 2 context lengths: uniform in [1200, 1300]."""
    return [int(x) for x in randint(seed, 7, batch, 1200, 1301)]


def config2_batch(seed: int = 2) -> VerifyBatch:
    """BASELINE config 2 attention inputs: b8 bf16, L ~ U[1200,1300], K=8."""
    return verify_batch(seed, config2_ctx_lens(seed), [9] * 8, num_blocks=64, dtype="bf16")


def config3_prompts(batch: int, seed: int = 3, prefix: int = 1200, span: int = 40, vocab: int = 151936):
    """BASELINE config 3 prompts: a 1200-token document made of 40-token
    spans that recur across it (span i at chapter positions i and 7i mod N,
    after benchmarks/rag_bench.py:80-105), followed per request by the
    first tokens of one span as the question, so an answer quoting the
    document is n-gram draftable."""
    nspans = 12
    spans = [[int(x) for x in randint(seed, 90 + i, span, 100, vocab)] for i in range(nspans)]
    doc = []
    i = 0
    while len(doc) < prefix:
        doc += spans[i % nspans] + spans[(i * 7) % nspans][: span // 4]
        i += 1
    doc = doc[:prefix]
    return [doc + spans[(b * 5 + 1) % nspans][:6] for b in range(batch)]
