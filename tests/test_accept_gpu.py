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


# Rows cut into chunks longer than one slab: the statistics pass rescales its
# running sum when a later slab raises the chunk maximum, and the argmax
# passes compare keys across slabs.  V = 300000 with few rows takes the
# narrow slabs (128 chunks of 2344 elements: slabs of 2048 + 296); V = 1.1M
# with 9 rows takes the wide ones (128 chunks of 8600: slabs of 8192 + 408).
def slab_of(V):
    """The slab length these tests' row counts select: narrow below 1M, wide above."""
    return 2048 if V < 10 ** 6 else 8192


def plant_second_slabs(x, V, seed):
    """Large values in the second slab of some chunks (the maximum of those
    chunks arrives after the first slab) and an exact tie between the two
    slabs of another chunk."""
    per = ((V + 127) // 128 + 7) & ~7
    slab = slab_of(V)
    rng = np.random.default_rng(seed)
    for r in range(x.shape[0]):
        for c in rng.choice(127, 6, replace=False):  # the last chunk is short: it may hold one slab only
            x[r, c * per + slab + int(rng.integers(0, per - slab))] = 8.0 + rng.random()
        c = int(rng.integers(0, 127))
        x[r, c * per + 3] = x[r, c * per + slab + 5] = 12.0  # equal row maxima in both slabs: the first index wins
    return x


@pytest.mark.parametrize("dtype,V", [("bf16", 300000), ("f32", 300000), ("bf16", 1100000)])
def test_greedy_multi_slab_chunks(dtype, V):
    print(f"case: greedy multi-slab {dtype} V={V}", flush=True)
    K = 2 if V < 10 ** 6 else 8
    B = 2 if V < 10 ** 6 else 1
    x = plant_second_slabs(synth.normal(70, 71, B * (K + 1) * V, 2.0).reshape(B * (K + 1), V), V, 72)
    per = ((V + 127) // 128 + 7) & ~7
    x[1, 40 * per + slab_of(V) + 1] = np.nan  # in a second slab; NaN beats every number
    lg = torch.from_numpy(x.astype(np.float32)).cuda().to(TDT[dtype])
    am = [oa.argmax_first(r) for r in host(lg)]
    lists = [am[b * (K + 1): b * (K + 1) + K - b] + ([] if b == 0 else [7]) for b in range(B)]
    d, nd = pad(lists, K)
    got = results(*accept_greedy(lg, d, nd, K + 1))
    assert got == oa.greedy_round(lists, host(lg), K + 1)
    assert am[1] == 40 * per + slab_of(V) + 1


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_stochastic_multi_slab_chunks(dtype):
    # model drafts, B = 2, K = 2 (10 statistics rows: the narrow slabs), then an n-gram batch at V = 1.1M (wide)
    print(f"case: stochastic multi-slab {dtype}", flush=True)
    B, K, V = 2, 2, 300000
    dl, tl, lists = model_case(73, B, K, V, dtype)
    tl = torch.from_numpy(plant_second_slabs(host(tl), V, 74).astype(np.float32)).cuda().to(TDT[dtype])
    dl = torch.from_numpy(plant_second_slabs(host(dl), V, 74).astype(np.float32)).cuda().to(TDT[dtype])
    u, q = draw_randomness([len(x) for x in lists], V, TDT[dtype], "cuda", True,
                           torch.Generator(device="cuda").manual_seed(75))
    d, nd = pad(lists, K)
    got = results(*accept_stochastic(tl, d, nd, torch.tensor([1.0, 0.8], device="cuda"), q, uniforms=u,
                                     draft_logits=dl, target_seq_stride=K + 1, draft_seq_stride=K + 1,
                                     draft_row_stride=1))
    T, D, U, Q = host(tl), host(dl), u.cpu().numpy(), host(q)
    for b, drafts in enumerate(lists):
        k = len(drafts)
        want = oa.verify_stochastic(drafts, T[b * (K + 1): b * (K + 1) + k + 1], D[b * (K + 1): b * (K + 1) + k],
                                    [1.0, 0.8][b], U[b, :k], Q[b], dtype)
        assert got[b] == want, (b, got[b], want)

    K, V = 8, 1100000
    tl = torch.from_numpy(plant_second_slabs(synth.normal(76, 77, (K + 1) * V, 2.0).reshape(K + 1, V), V, 78)
                          .astype(np.float32)).cuda().to(TDT[dtype])
    am = tl.argmax(-1).tolist()
    lists = [am[:K]]
    _, q = draw_randomness([K], V, TDT[dtype], "cuda", False, torch.Generator(device="cuda").manual_seed(79))
    d, nd = pad(lists, K)
    got = results(*accept_stochastic(tl, d, nd, torch.tensor([0.5], device="cuda"), q, target_seq_stride=K + 1))
    want = oa.verify(lists[0], host(tl), None, 0.5, None, host(q)[0], dtype)
    assert got[0] == want


def test_sampler_multi_slab_chunks():
    print("case: sampler multi-slab", flush=True)
    B, V = 4, 300000
    x = plant_second_slabs(synth.normal(80, 81, B * V, 2.0).reshape(B, V), V, 82)
    lg = torch.from_numpy(x.astype(np.float32)).cuda().to(torch.bfloat16)
    temps = torch.tensor([1.0, 0.0, 0.6, 1.5], device="cuda")
    q = torch.empty(B, V, device="cuda").exponential_(1, generator=torch.Generator(device="cuda").manual_seed(83))
    q.clamp_min_(1e-10)
    assert sample(lg, temps, q).tolist() == oa.sample_rows(host(lg), temps.cpu().numpy(), q.cpu().numpy())


# More drafts than 32: rows 33..63 of a sequence take lanes 33..63 of the
# accept walks' ballots.
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_long_draft_lists(dtype):
    print(f"case: K=40 {dtype}", flush=True)
    B, K, V = 3, 40, 5000
    # greedy: all 40 accepted + bonus, 37 accepted, none
    lg = logits_tensor(90, B * (K + 1), V, dtype)
    am = lg.argmax(-1).tolist()
    lists = [am[0:40], am[41:41 + 37] + [(am[41 + 37] + 1) % V] + am[41 + 38:41 + 40], [(am[82] + 1) % V] * 40]
    d, nd = pad(lists, K)
    got = results(*accept_greedy(lg, d, nd, K + 1))
    assert got == oa.greedy_round(lists, host(lg), K + 1)
    assert [len(g) for g in got] == [41, 38, 1]
    # stochastic, model drafts: identical draft and target rows accept all 40 + bonus
    for identical in (True, False):
        dl, tl, lists = model_case(91, B, K, V, dtype, identical)
        u, q = draw_randomness([len(x) for x in lists], V, TDT[dtype], "cuda", True,
                               torch.Generator(device="cuda").manual_seed(92))
        d, nd = pad(lists, K)
        got = results(*accept_stochastic(tl, d, nd, torch.ones(B, device="cuda"), q, uniforms=u, draft_logits=dl,
                                         target_seq_stride=K + 1, draft_seq_stride=K + 1, draft_row_stride=1))
        T, D, U, Q = host(tl), host(dl), u.cpu().numpy(), host(q)
        for b, drafts in enumerate(lists):
            k = len(drafts)
            want = oa.verify_stochastic(drafts, T[b * (K + 1): b * (K + 1) + k + 1], D[b * (K + 1): b * (K + 1) + k],
                                        1.0, U[b, :k], Q[b], dtype)
            assert got[b] == want, (identical, b, got[b], want)
        if identical:
            assert [len(g) for g in got] == [len(x) + 1 for x in lists] and len(got[0]) == 41
    # stochastic, n-gram drafts on peaked rows: the target samples match the drafts far past 32
    x = synth.normal(93, 94, B * (K + 1) * V, 1.0).reshape(B * (K + 1), V)
    peak = [int(v) for v in synth.randint(95, 96, B * (K + 1), 0, V)]
    x[np.arange(B * (K + 1)), peak] = 40.0
    tl = torch.from_numpy(x.astype(np.float32)).cuda().to(TDT[dtype])
    lists = [peak[0:40], peak[41:41 + 35] + [(peak[41 + 35] + 1) % V], peak[82:82 + 12]]
    _, q = draw_randomness([len(x) for x in lists], V, TDT[dtype], "cuda", False,
                           torch.Generator(device="cuda").manual_seed(97))
    d, nd = pad(lists, K)
    got = results(*accept_stochastic(tl, d, nd, torch.tensor([1.0, 1.0, 0.9], device="cuda"), q,
                                     target_seq_stride=K + 1))
    T, Q = host(tl), host(q)
    for b, drafts in enumerate(lists):
        want = oa.verify(drafts, T[b * (K + 1): b * (K + 1) + len(drafts) + 1], None, [1.0, 1.0, 0.9][b], None,
                         Q[b, :len(drafts) + 1], dtype)
        assert got[b] == want, (b, got[b], want)
    assert len(got[0]) == 41 and len(got[1]) == 36


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_accept_ratio_boundaries_multi_slab(dtype):
    # Uniforms a hair below (accept) and above (reject) each draft's min(1, p_t/p_d), on rows whose
    # statistics take two slabs per chunk with maxima planted in the second: every decision pins the
    # ratio, and with it both rows' fp64 sums, to the dtype's resolution.  Call i accepts drafts
    # 0..i-1 and rejects draft i (the last call accepts all).
    print(f"case: ratio boundaries {dtype}", flush=True)
    B, K, V = 3, 3, 300000
    temps = [1.0, 0.8, 1.3]
    T = plant_second_slabs(synth.normal(100, 101, B * (K + 1) * V, 2.0).reshape(B * (K + 1), V), V, 102)
    D = plant_second_slabs(synth.normal(103, 104, B * K * V, 2.0).reshape(B * K, V), V, 105)
    tl = torch.from_numpy(T.astype(np.float32)).cuda().to(TDT[dtype])
    dl = torch.from_numpy(D.astype(np.float32)).cuda().to(TDT[dtype])
    T, D = host(tl), host(dl)
    floor = float(oa.round_to(1e-20, dtype))
    lists, ratio = [], np.zeros((B, K))
    for b in range(B):
        pt = oa.softmax_rows(T[b * (K + 1): b * (K + 1) + K], temps[b], dtype)
        pd = oa.softmax_rows(D[b * K: (b + 1) * K], temps[b], dtype)
        toks = []
        for i in range(K):
            r = oa.div_round(pt[i], np.maximum(pd[i], floor), dtype)
            cand = np.flatnonzero((r > 0.05) & (r < 0.95))
            toks.append(int(cand[(7 * b + 3 * i) % len(cand)]))
            ratio[b, i] = r[toks[-1]]
        lists.append(toks)
    q = torch.empty(B, V, dtype=TDT[dtype], device="cuda").exponential_(
        1, generator=torch.Generator(device="cuda").manual_seed(106))
    d, nd = pad(lists, K)
    for i in range(K + 1):
        u = np.full((B, K), 0.5, dtype=np.float32)
        u[:, :i] = (ratio[:, :i] * (1 - 2 ** -14)).astype(np.float32)
        if i < K:
            u[:, i] = (ratio[:, i] * (1 + 2 ** -14)).astype(np.float32)
        got = results(*accept_stochastic(tl, d, nd, torch.tensor(temps, device="cuda"), q,
                                         uniforms=torch.from_numpy(u).cuda(), draft_logits=dl,
                                         target_seq_stride=K + 1, draft_seq_stride=K, draft_row_stride=1))
        for b in range(B):
            want = oa.verify_stochastic(lists[b], T[b * (K + 1): (b + 1) * (K + 1)], D[b * K: (b + 1) * K],
                                        temps[b], u[b], host(q)[b], dtype)
            assert len(want) == i + 1
            assert got[b] == want, (i, b, got[b], want)


# Rows whose start is not 16-byte aligned (V odd: every other row of a bf16 batch, and V not a
# multiple of 4 for fp32) take the element-by-element slab loads; V not a multiple of 8 leaves a
# partial last group in every row.
@pytest.mark.parametrize("dtype,V", [("bf16", 30001), ("f32", 30002), ("bf16", 1001)])
def test_unaligned_rows(dtype, V):
    print(f"case: unaligned rows {dtype} V={V}", flush=True)
    B, K = 3, 4
    # greedy
    lg = logits_tensor(110, B * (K + 1), V, dtype)
    am = lg.argmax(-1).tolist()
    lists = [am[0:4], am[5:7] + [(am[7] + 1) % V], []]
    d, nd = pad(lists, K)
    got = results(*accept_greedy(lg, d, nd, K + 1))
    assert got == oa.greedy_round(lists, host(lg), K + 1)
    # stochastic, model drafts
    dl, tl, lists = model_case(111, B, K, V, dtype)
    u, q = draw_randomness([len(x) for x in lists], V, TDT[dtype], "cuda", True,
                           torch.Generator(device="cuda").manual_seed(112))
    d, nd = pad(lists, K)
    got = results(*accept_stochastic(tl, d, nd, torch.tensor([1.0, 0.7, 1.0], device="cuda"), q, uniforms=u,
                                     draft_logits=dl, target_seq_stride=K + 1, draft_seq_stride=K + 1,
                                     draft_row_stride=1))
    T, D, U, Q = host(tl), host(dl), u.cpu().numpy(), host(q)
    for b, drafts in enumerate(lists):
        k = len(drafts)
        want = oa.verify_stochastic(drafts, T[b * (K + 1): b * (K + 1) + k + 1], D[b * (K + 1): b * (K + 1) + k],
                                    [1.0, 0.7, 1.0][b], U[b, :k], Q[b], dtype)
        assert got[b] == want, (b, got[b], want)
    # stochastic, n-gram drafts (noise rows [K+1, V] per sequence, also unaligned)
    am = tl.argmax(-1).tolist()
    lists = [am[0:4], am[5:6], am[10:13]]
    _, q = draw_randomness([len(x) for x in lists], V, TDT[dtype], "cuda", False,
                           torch.Generator(device="cuda").manual_seed(113))
    d, nd = pad(lists, K)
    got = results(*accept_stochastic(tl, d, nd, torch.tensor([0.9, 1.0, 1.1], device="cuda"), q,
                                     target_seq_stride=K + 1))
    for b, drafts in enumerate(lists):
        want = oa.verify(drafts, T[b * (K + 1): b * (K + 1) + len(drafts) + 1], None, [0.9, 1.0, 1.1][b], None,
                         host(q)[b, :len(drafts) + 1], dtype)
        assert got[b] == want, (b, got[b], want)
    # the sampler over the same rows (fp32 noise [B, V])
    rows = tl[:B]
    temps = torch.tensor([1.0, 0.0, 0.6], device="cuda")
    qn = torch.empty(B, V, device="cuda").exponential_(1, generator=torch.Generator(device="cuda").manual_seed(114))
    qn.clamp_min_(1e-10)
    assert sample(rows, temps, qn).tolist() == oa.sample_rows(host(rows), temps.cpu().numpy(), qn.cpu().numpy())
