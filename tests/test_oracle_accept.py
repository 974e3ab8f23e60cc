"""Pins the CPU acceptance oracle (oracle/accept.py) before any GPU result is
compared with it: torch's own sampling routine, the torch-executed
reference algorithm with the same random stream, and closed-form cases."""

import numpy as np
import pytest
import torch

from oracle import accept as oa
from oracle.torch_cpu import sample as sampler_torch
from oracle.torch_cpu import verify_stochastic as reference_torch

TDT = {"bf16": torch.bfloat16, "f32": torch.float32}


def draw_noise(K, V, dtype, g, with_draft_rows):
    """What the reference draws from its generator, in its order: rand(K),
    then the exponential noise of its single multinomial call."""
    if with_draft_rows:
        u = torch.rand(K, generator=g)
        q = torch.empty(V, dtype=TDT[dtype]).exponential_(1, generator=g)
        return u.numpy(), q.float().numpy()
    q = torch.empty(K + 1, V, dtype=TDT[dtype]).exponential_(1, generator=g)
    return None, q.float().numpy()


def case(seed, K, V, dtype, sigma=2.0, corr=0.5, identical=False):
    gen = torch.Generator().manual_seed(seed)
    dl = torch.randn(K + 1, V, generator=gen) * sigma
    tl = dl.clone() if identical else dl + corr * torch.randn(K + 1, V, generator=gen)
    dl, tl = dl.to(TDT[dtype]), tl.to(TDT[dtype])
    pd = torch.softmax(dl[:K].float(), -1)
    drafts = [int(torch.multinomial(pd[i], 1, generator=gen)) for i in range(K)]
    return drafts, tl, dl[:K]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_multinomial_is_argmax_over_exponential_noise(dtype):
    # the identity the oracle (and the GPU kernel) rely on, checked against
    # torch's own multinomial with the generator state cloned
    for seed in range(40):
        p = torch.softmax(torch.randn(3, 4096, generator=torch.Generator().manual_seed(seed)) * 2, -1).to(TDT[dtype])
        g1, g2 = torch.Generator().manual_seed(seed), torch.Generator().manual_seed(seed)
        want = torch.multinomial(p, 1, generator=g1).squeeze(1).tolist()
        q = torch.empty_like(p).exponential_(1, generator=g2)
        got = [oa.multinomial(p[r].float().numpy(), q[r].float().numpy(), dtype) for r in range(3)]
        assert got == want


def test_argmax_first_matches_torch_on_ties_and_nan():
    rng = np.random.default_rng(0)
    for _ in range(200):
        v = rng.integers(-3, 4, size=64).astype(np.float32)  # many ties
        if rng.random() < 0.2:
            v[rng.integers(0, 64, size=2)] = np.nan
        assert oa.argmax_first(v) == int(torch.from_numpy(v).argmax())
    assert oa.argmax_first(np.full(5, -np.inf)) == int(torch.full((5,), -float("inf")).argmax())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_greedy_round_matches_torch_argmax_walk(dtype):
    rng = np.random.default_rng(1)
    K, V = 8, 1000
    for trial in range(30):
        logits = torch.from_numpy(np.round(rng.normal(size=(4 * (K + 1), V)) * 2)).to(TDT[dtype])  # rounded: ties
        am = logits.argmax(-1).tolist()
        drafts = []
        for b in range(4):
            k = int(rng.integers(1, K + 1))
            acc = int(rng.integers(0, k + 1))
            d = am[b * (K + 1): b * (K + 1) + acc] + list(rng.integers(0, V, size=k - acc))
            drafts.append([int(x) for x in d])
        got = oa.greedy_round(drafts, logits.float().numpy(), stride=K + 1)
        for b, d in enumerate(drafts):
            row = am[b * (K + 1): b * (K + 1) + len(d) + 1]
            want = []
            for j, t in enumerate(d):
                if t != row[j]:
                    want.append(row[j])
                    break
                want.append(t)
            else:
                want.append(row[len(d)])
            assert got[b] == want


def test_greedy_closed_forms():
    # every draft accepted -> K drafts + bonus; first mismatch -> stop there
    assert oa.verify_greedy([5, 6, 7], [5, 6, 7, 9]) == [5, 6, 7, 9]
    assert oa.verify_greedy([5, 6, 7], [5, 1, 7, 9]) == [5, 1]
    assert oa.verify_greedy([5], [4, 9]) == [4]
    assert oa.verify_greedy([], [3]) == [3]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("mode", ["model", "ngram"])
def test_stochastic_oracle_reproduces_torch_execution(dtype, mode):
    # same generator stream on both sides; V small enough to run many seeds
    K, V = 8, 4096
    for seed in range(25):
        drafts, tl, dl = case(seed, K, V, dtype, identical=(seed % 5 == 0))
        drows = dl if mode == "model" else None
        g1, g2 = torch.Generator().manual_seed(100 + seed), torch.Generator().manual_seed(100 + seed)
        want = reference_torch(drafts, tl, drows, 1.0, g1)
        u, q = draw_noise(K, V, dtype, g2, mode == "model")
        got = oa.verify_stochastic(drafts, tl.float().numpy(), None if drows is None else drows.float().numpy(),
                                   1.0, u, q, dtype)
        assert got == want, (seed, got, want)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("mode", ["model", "ngram"])
def test_stochastic_oracle_full_vocab(dtype, mode):
    # config 2's distributions at the full vocabulary: the exact-then-rounded
    # softmax of the oracle (and the GPU kernels) against torch's own fp32
    # softmax executing the reference's call sequence, 12 seeds per mode
    K, V = 8, 151936
    for seed in range(12):
        drafts, tl, dl = case(seed, K, V, dtype)
        drows = dl if mode == "model" else None
        g1, g2 = torch.Generator().manual_seed(7 + seed), torch.Generator().manual_seed(7 + seed)
        want = reference_torch(drafts, tl, drows, 1.0, g1)
        u, q = draw_noise(K, V, dtype, g2, mode == "model")
        got = oa.verify_stochastic(drafts, tl.float().numpy(), None if drows is None else drows.float().numpy(), 1.0,
                                   u, q, dtype)
        assert got == want, (seed, got, want)


def test_stochastic_closed_forms():
    V, K = 64, 3
    rng = np.random.default_rng(3)
    x = rng.normal(size=(K + 1, V))
    q = rng.exponential(size=V)
    # draft == target distribution: every ratio is 1, so u < 1 accepts all; the bonus is
    # multinomial(p_t[K]) = argmax(p_t[K] / q)
    out = oa.verify_stochastic([1, 2, 3], x, x[:K], 1.0, [0.999, 0.5, 0.0], q, "f32")
    p = oa.softmax_rows(x, 1.0, "f32")
    assert out == [1, 2, 3, int(np.argmax(p[K].astype(np.float32) / q.astype(np.float32)))]
    # a draft the target cannot produce (p_t = 0) is always rejected, and the resample
    # never returns it (its residual is 0)
    xt = x.copy()
    xt[0, 7] = -1e4
    out = oa.verify_stochastic([7, 2, 3], xt, x[:K], 1.0, [0.0, 0.0, 0.0], q, "f32")
    assert len(out) == 1 and out[0] != 7
    # temperature <= 1e-6 dispatches to greedy (rejection_sampler.py:95)
    assert oa.verify([int(np.argmax(x[0])), 0], x[:3], temperature=0.0)[0] == int(np.argmax(x[0]))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sampler_oracle_reproduces_torch_execution(dtype):
    # 40 seeds x 6 rows of V = 4096 with mixed temperatures (greedy rows among them)
    temps = torch.tensor([1.0, 0.0, 0.6, 1.7, 1e-7, 1.0])
    for seed in range(40):
        g = torch.Generator().manual_seed(seed)
        lg = (torch.randn(6, 4096, generator=g) * 2.0).to(TDT[dtype])
        q = torch.empty(6, 4096).exponential_(1, generator=g).clamp_min_(1e-10)
        want = sampler_torch(lg, temps, q).tolist()
        got = oa.sample_rows(lg.float().numpy().astype(np.float64), temps.numpy(), q.numpy())
        assert got == want, seed


def test_sampler_closed_forms():
    # greedy rows ignore the noise; a one-hot-dominant row samples its peak whatever the noise;
    # equal logits sample argmin(noise) (p uniform, so argmax(p / q) = argmin q)
    x = np.zeros(50)
    x[7] = 80.0
    q = np.linspace(0.5, 3.0, 50)
    assert oa.sample(x, 0.0, q) == 7 and oa.sample(x, 1.0, q) == 7
    flat = np.ones(50)
    q2 = np.full(50, 2.0)
    q2[31] = 0.1
    assert oa.sample(flat, 1.0, q2) == 31
    assert oa.sample(flat, 0.0, q2) == 0  # argmax ties: first index
