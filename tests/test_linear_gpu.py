"""The few-row linear kernel (nsv_linear) against plain PyTorch fp32
restatements of the ops it replaces or fuses: F.linear (layers/linear.py),
residual RMSNorm (layers/layernorm.py:18-35) as its prologue, SiluAndMul
(layers/activation.py:17-19) and the residual add as its epilogues.

Tolerances: every output is one bf16 rounding of an fp32 result, held to
the bf16 contract (2e-2 abs / 1e-2 rel) with operands scaled so outputs are
O(1).  With the RMSNorm prologue the kernel evaluates rmsnorm(r) * w @ W^T
as inv_rms(r) * (r @ W'^T) with W' = bf16(W * w) (the norm weight folded
into the weight rows), and the restatement follows that formulation; a
test below also holds it to the reference's order (normalised activation
rounded to bf16, then the product) within the same tolerance.  The
residual stream is checked against bf16(bf16(x W^T) + r) and the partial
sums of squares against the fp32 sums of the returned stream over each
16-column tile."""

import pytest
import torch
import torch.nn.functional as F

from naivllm_amd import _lib
from naivllm_amd.layers import qwen3 as qm

pytestmark = pytest.mark.gpu

BF16 = dict(atol=2e-2, rtol=1e-2)

# (M, N, K): Qwen3-0.6B projections at b1 / b2 / b8, an 8B projection, more
# rows than one workgroup row-chunk (80), a reduction that is not a
# multiple of the 1024-element wave round, and the test model's shapes
SHAPES = [(9, 4096, 1024), (18, 1024, 2048), (72, 6144, 1024), (72, 1024, 3072), (16, 6144, 4096),
          (100, 512, 1024), (1, 256, 256), (37, 2048, 264)]


def gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def randn(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g, device="cuda") * scale).to(torch.bfloat16)


def partial_squares(r: torch.Tensor, tiles: int) -> torch.Tensor:
    """[tiles, M] fp32 partial sums of r^2, as a residual epilogue writes them."""
    M, K = r.shape
    return r.float().pow(2).view(M, tiles, K // tiles).sum(-1).t().contiguous()


def norm_ref(r: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """The reference's order: bf16(rmsnorm(r) * w), the activation the projection consumes."""
    rf = r.float()
    return (rf / torch.sqrt(rf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).to(torch.bfloat16).float()


def norm_linear_ref(r: torch.Tensor, w: torch.Tensor, W: torch.Tensor, eps: float) -> torch.Tensor:
    """The kernel's order: inv_rms(r) * (r @ bf16(W * w)^T), fp32."""
    rf = r.float()
    inv = torch.rsqrt(rf.pow(2).mean(-1, keepdim=True) + eps)
    return inv * (rf @ (W.float() * w.float()).to(torch.bfloat16).float().t())


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("norm", [False, True])
def test_linear_plain(M, N, K, norm):
    print(f"case: linear plain M={M} N={N} K={K} norm={norm}", flush=True)
    g = gen(M * 31 + N + K)
    x = randn(g, M, K)
    w = randn(g, N, K, scale=K ** -0.5)
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    if norm:
        nw = (1.0 + 0.3 * torch.randn(K, generator=g, device="cuda")).to(torch.bfloat16)
        tiles = 8 if K % 8 == 0 else 1
        qm.linear(x, w, y, norm_w=nw, ss_in=partial_squares(x, tiles), eps=1e-6)
        torch.testing.assert_close(y.float(), norm_linear_ref(x, nw, w, 1e-6), **BF16)
        # the reference's rounding order lands within the same contract
        torch.testing.assert_close(y.float(), norm_ref(x, nw, 1e-6) @ w.float().t(), **BF16)
    else:
        qm.linear(x, w, y)
        torch.testing.assert_close(y.float(), x.float() @ w.float().t(), **BF16)


# I >= 2080 puts more than 256 16-column tiles on the grid, which takes the
# 32-column tiles (16 gate + 16 up rows); (9, 12288, 4096) and (20, 12288,
# 4096) run them with half chunks (two workgroups per CU at 9 rows, one at
# 20); 90 rows take two row blocks
@pytest.mark.parametrize("M,I,K,norm", [(9, 3072, 1024, True), (72, 3072, 1024, True), (5, 128, 256, True),
                                        (90, 256, 512, True), (40, 256, 1024, True), (18, 3072, 1024, True),
                                        (36, 3072, 1024, False), (50, 3072, 1024, True), (90, 3072, 1024, True),
                                        (1, 3072, 1024, False), (9, 12288, 4096, True), (20, 12288, 4096, True)])
def test_linear_swiglu(M, I, K, norm):
    print(f"case: linear swiglu M={M} I={I} K={K} norm={norm}", flush=True)
    g = gen(M + I + K)
    r = randn(g, M, K)
    w = randn(g, 2 * I, K, scale=K ** -0.5)
    y = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    if norm:
        nw = (1.0 + 0.3 * torch.randn(K, generator=g, device="cuda")).to(torch.bfloat16)
        qm.linear(r, w, y, norm_w=nw, ss_in=partial_squares(r, 4), eps=1e-6, swiglu=True)
        gu = norm_linear_ref(r, nw, w, 1e-6).to(torch.bfloat16).float()  # the bf16 gate_up tensor
    else:
        qm.linear(r, w, y, swiglu=True)
        gu = (r.float() @ w.float().t()).to(torch.bfloat16).float()
    want = F.silu(gu[:, :I]) * gu[:, I:]
    torch.testing.assert_close(y.float(), want, **BF16)


def bf16_of_magnitudes(g, n, lo_exp, hi_exp):
    """n bf16 values of random sign, exponent in [lo_exp, hi_exp) and mantissa."""
    e = torch.randint(lo_exp, hi_exp, (n,), generator=g, device="cuda").float()
    f = 1.0 + torch.randint(0, 128, (n,), generator=g, device="cuda").float() / 128
    s = torch.where(torch.rand(n, generator=g, device="cuda") < 0.5, -1.0, 1.0)
    return (s * f * torch.exp2(e)).to(torch.bfloat16)


@pytest.mark.parametrize("lo_exp,hi_exp", [(-8, 8), (-110, -100), (118, 128)])
def test_output_rounding_is_round_to_nearest_even(lo_exp, hi_exp):
    # y[m][n] = s[n] + t[m] from two unit products: the fp32 sum of two bf16
    # values (ties, sticky bits and, near the top of the range, overflow to
    # inf among them) rounded once to bf16, bit for bit as torch rounds the
    # same fp32 value
    print(f"case: output rounding exponents [{lo_exp}, {hi_exp})", flush=True)
    M, N, K = 16, 256, 32
    g = gen(lo_exp * 131 + hi_exp)
    s = bf16_of_magnitudes(g, N, lo_exp, hi_exp)
    t = bf16_of_magnitudes(g, M, lo_exp - 9, hi_exp)  # exponent gaps up to 9 + the range: ties and sticky bits
    x = torch.zeros(M, K, dtype=torch.bfloat16, device="cuda")
    x[:, 0] = 1.0
    x[:, 1] = t
    w = torch.zeros(N, K, dtype=torch.bfloat16, device="cuda")
    w[:, 0] = s
    w[:, 1] = 1.0
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    qm.linear(x, w, y)
    want = (s.float().cpu()[None, :] + t.float().cpu()[:, None]).to(torch.bfloat16)
    got = y.cpu()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (got - want).abs().max()


# (4-column tiles: 1, 9, 16, 18 and 31 rows, reductions of whole and partial 128-element chunks, 1-3 per wave)
@pytest.mark.parametrize("M,N,K", [(9, 1024, 2048), (18, 1024, 3072), (72, 1024, 3072), (100, 256, 512),
                                   (3, 4096, 4096), (1, 1024, 3072), (16, 1024, 1032), (31, 512, 2056)])
def test_linear_residual(M, N, K):
    print(f"case: linear residual M={M} N={N} K={K}", flush=True)
    g = gen(M * 7 + N * 3 + K)
    x = randn(g, M, K)
    w = randn(g, N, K, scale=K ** -0.5)
    r0 = randn(g, M, N)
    r = r0.clone()
    rows = qm.ss_rows(M, N, K)  # one per 16-column tile, or 8-column tile (9 x 1024 x 2048)
    ss = torch.full((rows, M), float("nan"), device="cuda")
    qm.linear(x, w, resid=r, ss_out=ss)
    prod = (x.float() @ w.float().t()).to(torch.bfloat16)
    torch.testing.assert_close(r.float(), (prod.float() + r0.float()).to(torch.bfloat16).float(), **BF16)
    torch.testing.assert_close(ss, partial_squares(r, rows), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("M", [9, 18])
def test_linear_chain_matches_unfused_layer(M):
    # o_proj (residual epilogue) -> gate_up (RMSNorm prologue, SwiGLU) ->
    # down (residual epilogue) -> LM head (RMSNorm prologue): the fused
    # chain of one decoder layer against the unfused bf16 sequence (up to 31
    # rows o_proj and down take 8-column tiles and write twice the partials)
    print(f"case: linear chain vs unfused layer M={M}", flush=True)
    g = gen(5)
    E, I, V = 1024, 3072, 4096
    o = randn(g, M, 2048)
    resid = randn(g, M, E)
    w_o = randn(g, E, 2048, scale=2048 ** -0.5)
    w_gu = randn(g, 2 * I, E, scale=E ** -0.5)
    w_d = randn(g, E, I, scale=I ** -0.5)
    w_lm = randn(g, V, E, scale=E ** -0.5)
    ln2 = (1.0 + 0.3 * torch.randn(E, generator=g, device="cuda")).to(torch.bfloat16)
    ln_f = (1.0 + 0.3 * torch.randn(E, generator=g, device="cuda")).to(torch.bfloat16)

    r = resid.clone()
    ss_o = torch.empty(qm.ss_rows(M, E, 2048), M, device="cuda")
    ss_d = torch.empty(qm.ss_rows(M, E, I), M, device="cuda")
    act = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    logits = torch.empty(M, V, dtype=torch.bfloat16, device="cuda")
    qm.linear(o, w_o, resid=r, ss_out=ss_o)
    qm.linear(r, w_gu, act, norm_w=ln2, ss_in=ss_o, swiglu=True)
    qm.linear(act, w_d, resid=r, ss_out=ss_d)
    qm.linear(r, w_lm, logits, norm_w=ln_f, ss_in=ss_d)

    bf = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
    x = bf(o.float() @ w_o.float().t())
    rr = bf(x + resid.float())
    gu = bf(norm_linear_ref(rr.to(torch.bfloat16), ln2, w_gu, 1e-6))
    a = bf(F.silu(gu[:, :I]) * gu[:, I:])
    rr = bf(bf(a @ w_d.float().t()) + rr)
    want = norm_linear_ref(rr.to(torch.bfloat16), ln_f, w_lm, 1e-6)
    rel = (logits.float() - want).norm() / want.norm()
    assert rel < 1e-2, float(rel)


@pytest.mark.parametrize("M,N,K", [(72, 1024, 2048), (48, 512, 3072), (33, 1024, 1024)])
def test_split_reduction_is_deterministic_and_reusable(M, N, K):
    # shapes whose reduction is split over several workgroups per column tile:
    # repeated calls on the shared workspace give identical bits (fixed-order
    # partial sums, counters left at zero), for every epilogue
    print(f"case: split-K linear M={M} N={N} K={K}", flush=True)
    from naivllm_amd import _lib
    assert _lib.lib().nsv_linear_workspace_size(M, N, K) > 0
    g = gen(M + N + K)
    x = randn(g, M, K)
    w = randn(g, N, K, scale=K ** -0.5)
    ys = [torch.empty(M, N, dtype=torch.bfloat16, device="cuda") for _ in range(3)]
    for y in ys:
        qm.linear(x, w, y)
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[1], ys[2])
    torch.testing.assert_close(ys[0].float(), x.float() @ w.float().t(), **BF16)
    r0 = randn(g, M, N)
    outs = []
    for _ in range(2):
        r = r0.clone()
        ss = torch.empty(qm.ss_rows(M, N, K), M, device="cuda")
        qm.linear(x, w, resid=r, ss_out=ss)
        outs.append((r, ss))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    prod = (x.float() @ w.float().t()).to(torch.bfloat16)
    torch.testing.assert_close(outs[0][0].float(), (prod.float() + r0.float()).to(torch.bfloat16).float(), **BF16)


# The streaming kernel nsv_linear takes for very wide plain projections (the
# LM head: at least 32 16-row tiles per CU), at the rows a verify round asks
# logits for (b1, b2, b8), the 8B head's reduction, and the row count past its
# LDS capacity at K = 1024 (80 rows: the 16-column kernel again).
WIDE = [(9, 151936, 1024), (1, 151936, 1024), (18, 151936, 1024), (72, 151936, 1024), (80, 151936, 1024),
        (9, 151936, 4096), (16, 135168, 2048)]


@pytest.mark.parametrize("M,N,K", WIDE)
def test_linear_wide(M, N, K):
    print(f"case: linear wide M={M} N={N} K={K}", flush=True)
    g = gen(M * 7 + N + K)
    x = randn(g, M, K)
    w = randn(g, N, K, scale=K ** -0.5)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    qm.linear(x, w, y)
    torch.testing.assert_close(y.float(), x.float() @ w.float().t(), **BF16)


# The LM head on its packed weight (nsv_lm_head_pack + nsv_lm_head): the
# packed copy is the permutation its header states (checked against torch's
# view/permute of the row-major weight), and the head's output has the same
# bits as nsv_linear's streaming dispatch on the row-major weight (the same
# MFMA operands in the same order), at every WIDE shape it takes; one row
# count past its limit is refused before any launch.
@pytest.mark.parametrize("M,N,K", [c for c in WIDE if c[0] <= (79 if c[2] == 1024 else 39 if c[2] == 2048 else 19)])
def test_lm_head_packed(M, N, K):
    print(f"case: lm head packed M={M} N={N} K={K}", flush=True)
    h = _lib.lib()
    rows = h.nsv_lm_head_rows(N, K)
    assert M <= rows
    g = gen(M * 11 + N + K)
    x = randn(g, M, K)
    w = randn(g, N, K, scale=K ** -0.5)
    packed = torch.full_like(w, float("nan"))
    assert h.nsv_lm_head_pack(w.data_ptr(), packed.data_ptr(), N, K, _lib.stream_ptr(w.device)) == 0
    want = w.view(N // 16, 16, K // 256, 8, 4, 8).permute(0, 2, 3, 4, 1, 5).reshape(N, K)
    assert torch.equal(packed, want)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    qm.lm_head(x, packed, y)
    y_ref = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    qm.linear(x, w, y_ref)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    torch.testing.assert_close(y.float(), x.float() @ w.float().t(), **BF16)
    big = torch.empty(rows + 1, K, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(rows + 1, N, dtype=torch.bfloat16, device="cuda")
    assert h.nsv_lm_head(big.data_ptr(), packed.data_ptr(), out.data_ptr(), rows + 1, N, K,
                         _lib.stream_ptr(w.device)) == -2


# The decode-shaped kernel (nsv_linear_decode): one or two rows, each
# epilogue, the Qwen3-0.6B projections and an 8B-wide reduction; the same
# contract against the same fp32 restatements (its reduction order is its own)
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("N,K,norm", [(4096, 1024, False), (4096, 1024, True), (1024, 2048, False),
                                      (6144, 4096, True)])
def test_linear_decode_plain(M, N, K, norm):
    print(f"case: linear decode plain M={M} N={N} K={K} norm={norm}", flush=True)
    g = gen(M * 13 + N + K)
    x = randn(g, M, K)
    w = randn(g, N, K, scale=K ** -0.5)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    if norm:
        nw = (1.0 + 0.3 * torch.randn(K, generator=g, device="cuda")).to(torch.bfloat16)
        qm.linear(x, w, y, norm_w=nw, ss_in=partial_squares(x, 256), eps=1e-6, decode=True)
        torch.testing.assert_close(y.float(), norm_linear_ref(x, nw, w, 1e-6), **BF16)
    else:
        qm.linear(x, w, y, decode=True)
        torch.testing.assert_close(y.float(), x.float() @ w.float().t(), **BF16)


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("I,K,norm", [(3072, 1024, True), (3072, 1024, False)])
def test_linear_decode_swiglu(M, I, K, norm):
    print(f"case: linear decode swiglu M={M} I={I} K={K} norm={norm}", flush=True)
    g = gen(M + I + K + 5)
    r = randn(g, M, K)
    w = randn(g, 2 * I, K, scale=K ** -0.5)
    y = torch.full((M, I), float("nan"), dtype=torch.bfloat16, device="cuda")
    if norm:
        nw = (1.0 + 0.3 * torch.randn(K, generator=g, device="cuda")).to(torch.bfloat16)
        qm.linear(r, w, y, norm_w=nw, ss_in=partial_squares(r, 64), eps=1e-6, swiglu=True, decode=True)
        gu = norm_linear_ref(r, nw, w, 1e-6).to(torch.bfloat16).float()
    else:
        qm.linear(r, w, y, swiglu=True, decode=True)
        gu = (r.float() @ w.float().t()).to(torch.bfloat16).float()
    torch.testing.assert_close(y.float(), F.silu(gu[:, :I]) * gu[:, I:], **BF16)


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("N,K", [(1024, 2048), (1024, 3072), (1040, 1024)])
def test_linear_decode_residual(M, N, K):
    # 1040 columns: the last workgroup holds 4 of them, as every other (N % 16 == 0)
    print(f"case: linear decode residual M={M} N={N} K={K}", flush=True)
    g = gen(M * 5 + N * 3 + K)
    x = randn(g, M, K)
    w = randn(g, N, K, scale=K ** -0.5)
    r0 = randn(g, M, N)
    r = r0.clone()
    rows = qm.decode_ss_rows(M, N)
    assert rows == N // 4
    ss = torch.full((rows, M), float("nan"), device="cuda")
    qm.linear(x, w, resid=r, ss_out=ss, decode=True)
    prod = (x.float() @ w.float().t()).to(torch.bfloat16)
    torch.testing.assert_close(r.float(), (prod.float() + r0.float()).to(torch.bfloat16).float(), **BF16)
    torch.testing.assert_close(ss, partial_squares(r, rows), rtol=1e-5, atol=1e-5)


def test_linear_decode_chain_feeds_prologue():
    # o_proj's decode partial sums (N / 4 slots) feed gate_up's decode prologue
    print("case: linear decode chain o_proj -> gate_up", flush=True)
    g = gen(77)
    M, E, I = 2, 1024, 3072
    a = randn(g, M, 2048)
    wo = randn(g, E, 2048, scale=2048 ** -0.5)
    wgu = randn(g, 2 * I, E, scale=E ** -0.5)
    nw = (1.0 + 0.3 * torch.randn(E, generator=g, device="cuda")).to(torch.bfloat16)
    r = randn(g, M, E)
    ss = torch.empty(qm.decode_ss_rows(M, E), M, device="cuda")
    qm.linear(a, wo, resid=r, ss_out=ss, decode=True)
    y = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    qm.linear(r, wgu, y, norm_w=nw, ss_in=ss, eps=1e-6, swiglu=True, decode=True)
    gu = norm_linear_ref(r, nw, wgu, 1e-6).to(torch.bfloat16).float()
    torch.testing.assert_close(y.float(), F.silu(gu[:, :I]) * gu[:, I:], **BF16)

