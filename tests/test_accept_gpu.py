"""GPU parity of the acceptance kernels against the CPU oracle: accepted
tokens must be identical on identical logits, uniforms and noise."""

import numpy as np
import pytest
import torch

from naivllm_amd.spec_engine import RejectionSampler
from naivllm_amd.spec_engine.rejection_sampler import accept_greedy, accept_stochastic, draw_randomness, sample
from naivllm_amd.utils import synth
from oracle import accept as oa
from oracle.torch_cpu import verify_stochastic as reference_torch

pytestmark = pytest.mark.gpu

TDT = {"bf16": torch.bfloat16, "f32": torch.float32}
V_FULL = 151936


def logits_tensor(seed, rows, V, dtype, std=2.0, device="cuda"):
    x = synth.normal(seed, 60, rows * V, std).reshape(rows, V)
    return torch.from_numpy(x.astype(np.float32)).to(device=device, dtype=TDT[dtype])


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


def pad(lists, K):
    d = torch.zeros(len(lists), K, dtype=torch.int32)
    for b, x in enumerate(lists):
        d[b, :len(x)] = torch.tensor(x, dtype=torch.int32)
    return d.cuda(), torch.tensor([len(x) for x in lists], dtype=torch.int32).cuda()


def results(tokens, lens):
    t, n = tokens.cpu().tolist(), lens.cpu().tolist()
    return [row[:k] for row, k in zip(t, n)]


def test_config1_greedy_fp32():
    # b1 fp32, 9 rows of 151936, drafts 0..4 equal the target argmax
    print("case: greedy config1", flush=True)
    K = 8
    lg = logits_tensor(1, K + 1, V_FULL, "f32")
    am = lg.argmax(-1).tolist()
    drafts = am[:5] + [int(x) for x in synth.randint(1, 61, 3, 0, V_FULL)]
    d, nd = pad([drafts], K)
    got = results(*accept_greedy(lg, d, nd, K + 1))
    want = oa.greedy_round([drafts], host(lg), K + 1)
    assert got == want
    assert len(got[0]) >= 6


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_greedy_batch_ragged_with_ties_and_nan(dtype):
    print(f"case: greedy ragged {dtype}", flush=True)
    B, K, V = 8, 8, 5000
    x = np.round(synth.normal(3, 62, B * (K + 1) * V, 1.5).reshape(B * (K + 1), V))  # integers: many ties
    x[5, 17] = np.nan
    x[5, 3000] = np.nan
    x[12, :] = -np.inf
    lg = torch.from_numpy(x.astype(np.float32)).cuda().to(TDT[dtype])
    am = [oa.argmax_first(r) for r in host(lg)]
    lists = []
    for b in range(B):
        k = [8, 0, 3, 8, 1, 5, 8, 2][b]
        acc = [8, 0, 1, 3, 1, 5, 0, 2][b]
        lists.append(am[b * (K + 1): b * (K + 1) + acc] + [int(v) for v in synth.randint(b, 63, k - acc, 0, V)])
    d, nd = pad(lists, K)
    got = results(*accept_greedy(lg, d, nd, K + 1))
    assert got == oa.greedy_round(lists, host(lg), K + 1)


def model_case(seed, B, K, V, dtype, identical=False):
    dl = logits_tensor(seed, B * (K + 1), V, dtype)
    tl = dl.clone() if identical else (dl.float() + 0.5 * logits_tensor(seed + 1, B * (K + 1), V, "f32", 1.0)).to(
        TDT[dtype])
    g = torch.Generator(device="cuda").manual_seed(seed)
    pd = torch.softmax(dl.float(), -1)
    lists = []
    for b in range(B):
        k = K - (b % 3)
        lists.append([int(torch.multinomial(pd[b * (K + 1) + i], 1, generator=g)) for i in range(k)])
    return dl, tl, lists


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("identical", [False, True])
def test_stochastic_model_drafts_config2(dtype, identical):
    # b8, target = draft + 0.5 N(0,1), drafts sampled from p_d
    print(f"case: stochastic model {dtype} identical={identical}", flush=True)
    B, K, V = 8, 8, V_FULL
    dl, tl, lists = model_case(4, B, K, V, dtype, identical)
    u, q = draw_randomness([len(x) for x in lists], V, TDT[dtype], "cuda", True,
                           torch.Generator(device="cuda").manual_seed(9))
    temp = torch.ones(B, device="cuda")
    d, nd = pad(lists, K)
    got = results(*accept_stochastic(tl, d, nd, temp, q, uniforms=u, draft_logits=dl, target_seq_stride=K + 1,
                                     draft_seq_stride=K + 1, draft_row_stride=1))
    T, D, U, Q = host(tl), host(dl), u.cpu().numpy(), host(q)
    for b, drafts in enumerate(lists):
        k = len(drafts)
        want = oa.verify_stochastic(drafts, T[b * (K + 1): b * (K + 1) + k + 1], D[b * (K + 1): b * (K + 1) + k], 1.0,
                                    U[b, :k], Q[b], dtype)
        assert got[b] == want, (b, got[b], want)
    if identical:
        assert all(len(g) == len(x) + 1 for g, x in zip(got, lists))  # every ratio is 1: all accepted + bonus


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_stochastic_ngram_mode_and_mixed_temperatures(dtype):
    print(f"case: stochastic ngram {dtype}", flush=True)
    B, K, V = 6, 8, 20000
    tl = logits_tensor(5, B * (K + 1), V, dtype)
    am = tl.argmax(-1).tolist()
    lists = [am[b * (K + 1): b * (K + 1) + [8, 4, 0, 8, 2, 6][b]] for b in range(B)]  # drafts = argmax
    temps = [1.0, 0.7, 1.0, 0.0, 1.3, 1e-7]
    active = [t > 1e-6 for t in temps]
    _, q = draw_randomness([len(x) for x in lists], V, TDT[dtype], "cuda", False,
                           torch.Generator(device="cuda").manual_seed(11), active=active)
    d, nd = pad(lists, K)
    got = results(*accept_stochastic(tl, d, nd, torch.tensor(temps, device="cuda"), q, target_seq_stride=K + 1))
    T, Q = host(tl), host(q)
    for b, drafts in enumerate(lists):
        k = len(drafts)
        rows = T[b * (K + 1): b * (K + 1) + k + 1]
        want = oa.verify(drafts, rows, None, temps[b], None, Q[b, :k + 1], dtype)
        assert got[b] == want, (b, got[b], want)


def test_residual_sum_zero_falls_back_to_target():
    # V = 3: p_d = softmax([0,0,0]) rounds to 0.333984 each in bf16; the target
    # logit -0.006 gives p_t(0) = 0.332 (< p_d(0)) while p_t(1), p_t(2) round to
    # p_d's value: ratio < 1, and the residual max(p_t - p_d, 0) is all zero, so the
    # resample draws from p_t (rejection_sampler.py:64-65)
    print("case: residual fallback", flush=True)
    tl = torch.tensor([[-0.006, 0.0, 0.0], [0.0, 0.0, 0.0]], dtype=torch.bfloat16, device="cuda")
    dl = torch.zeros(1, 3, dtype=torch.bfloat16, device="cuda")
    u = torch.tensor([[0.9999]], device="cuda")
    q = torch.tensor([[1.0, 0.5, 2.0]], dtype=torch.bfloat16, device="cuda")
    d, nd = pad([[0]], 1)
    got = results(*accept_stochastic(tl, d, nd, torch.ones(1, device="cuda"), q, uniforms=u, draft_logits=dl))
    want = oa.verify_stochastic([0], host(tl), host(dl), 1.0, [0.9999], host(q)[0], "bf16")
    p_t = oa.softmax_rows(host(tl), 1.0, "bf16")[0]
    p_d = oa.softmax_rows(host(dl), 1.0, "bf16")[0]
    assert p_t[0] < p_d[0] and np.all(oa.round_to(p_t - p_d, "bf16") <= 0)
    assert got == [want] and want == [1]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_drop_in_verify_matches_the_reference_torch_calls_on_gpu(dtype):
    # the reference's own torch calls, run by torch on the GPU with a seeded
    # generator, against RejectionSampler.verify with an identically seeded one
    print(f"case: drop-in verify {dtype}", flush=True)
    K, V = 8, V_FULL
    sampler = RejectionSampler()
    for seed in range(4):
        dl, tl, lists = model_case(20 + seed, 1, K, V, dtype, identical=(seed == 3))
        drafts = lists[0]
        for mode in ("model", "ngram"):
            drows = dl[:len(drafts)] if mode == "model" else None
            g1 = torch.Generator(device="cuda").manual_seed(100 + seed)
            g2 = torch.Generator(device="cuda").manual_seed(100 + seed)
            want = reference_torch(drafts, tl[:len(drafts) + 1], drows, 1.0, g1)
            got = sampler.verify(drafts, tl[:len(drafts) + 1], drows, 1.0, g2)
            assert got == want, (seed, mode, got, want)
    # greedy dispatch and the ready-token-list form
    lg = logits_tensor(30, K + 1, V, dtype)
    am = lg.argmax(-1).tolist()
    assert sampler.verify(am[:K], lg, temperature=0.0) == am
    assert sampler.verify_greedy(am[:3], am[:2] + [5, 6]) == am[:2] + [5]


def test_drop_in_strided_draft_rows():
    # the reference's fast path passes logit_buf[:, j, :] views of a (K, batch, V) buffer
    print("case: strided draft rows", flush=True)
    K, V, Bb = 8, 4096, 3
    buf = logits_tensor(40, K * Bb, V, "bf16").reshape(K, Bb, V)
    tl = logits_tensor(41, K + 1, V, "bf16")
    drafts = [int(x) for x in synth.randint(42, 0, K, 0, V)]
    g1, g2 = torch.Generator(device="cuda").manual_seed(5), torch.Generator(device="cuda").manual_seed(5)
    got = RejectionSampler().verify(drafts, tl, buf[:, 1, :], 1.0, g1)
    want = RejectionSampler().verify(drafts, tl, buf[:, 1, :].contiguous(), 1.0, g2)
    assert got == want


@pytest.mark.parametrize("dtype,V", [("bf16", V_FULL), ("f32", 5000), ("bf16", 300)])
def test_sampler_matches_oracle(dtype, V):
    # layers/sampler.py semantics: greedy rows take the argmax, the others
    # argmax(softmax(x / T) / q) in fp32; rows read through a row pitch of 2V
    print(f"case: sampler {dtype} V={V}", flush=True)
    B = 8
    lg = logits_tensor(7, 2 * B, V, dtype).view(B, 2 * V)[:, :V]
    temps = torch.tensor([1.0, 0.0, 0.5, 1.0, 2.0, 1e-7, 0.9, 1.0], device="cuda")
    q = torch.empty(B, V, device="cuda").exponential_(1, generator=torch.Generator(device="cuda").manual_seed(3))
    q.clamp_min_(1e-10)
    out = torch.full((B, 3), -1, dtype=torch.int32, device="cuda")
    sample(lg, temps, q, out=out[:, 1])
    got = out[:, 1].tolist()
    want = oa.sample_rows(host(lg), temps.cpu().numpy(), q.cpu().numpy())
    assert got == want
    assert out[:, 0].tolist() == [-1] * B and out[:, 2].tolist() == [-1] * B  # strided output only


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_stochastic_mixed_draft_modes(dtype):
    # a hybrid drafter's batch: sequences 0, 2, 5 carry model draft rows, the others n-gram drafts;
    # noise [B, K+1, V], row 0 of a model-mode sequence is its one multinomial
    print(f"case: stochastic mixed modes {dtype}", flush=True)
    B, K, V = 6, 8, 30000
    dl, tl, lists = model_case(12, B, K, V, dtype, False)
    mode = [1, 0, 1, 0, 0, 1]
    lists = [x[:k] for x, k in zip(lists, [8, 5, 3, 8, 0, 6])]
    g = torch.Generator(device="cuda").manual_seed(13)
    u = torch.rand(B, K, device="cuda", generator=g)
    q = torch.empty(B, K + 1, V, dtype=TDT[dtype], device="cuda").exponential_(1, generator=g)
    temps = torch.tensor([1.0, 1.0, 0.8, 0.0, 1.0, 1.2], device="cuda")
    d, nd = pad(lists, K)
    got = results(*accept_stochastic(tl, d, nd, temps, q, uniforms=u, draft_logits=dl, target_seq_stride=K + 1,
                                     draft_seq_stride=K + 1, draft_row_stride=1,
                                     draft_mode=torch.tensor(mode, dtype=torch.int32, device="cuda")))
    T, D, U, Q = host(tl), host(dl), u.cpu().numpy(), host(q)
    for b, drafts in enumerate(lists):
        k = len(drafts)
        rows = T[b * (K + 1): b * (K + 1) + k + 1]
        if mode[b]:
            want = oa.verify(drafts, rows, D[b * (K + 1): b * (K + 1) + k], float(temps[b]), U[b, :k], Q[b, 0], dtype)
        else:
            want = oa.verify(drafts, rows, None, float(temps[b]), None, Q[b, :k + 1], dtype)
        assert got[b] == want, (b, got[b], want)
