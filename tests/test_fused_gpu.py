"""The fused forward kernels (residual add + RMSNorm, the pre-attention
epilogue q/k RMSNorm + RoPE + paged KV store, SiLU * up) against plain
PyTorch fp32 restatements of the reference's ops (layers/layernorm.py:18-35,
layers/rotary_embedding.py:4-86, layers/attention.py:71-112,
layers/activation.py:17-19), and the whole Qwen3 verify forward against a
dense fp32 forward of the same weights.

Tolerances: each kernel output is one bf16 rounding of an fp32 result, so
it is held to the bf16 contract (2e-2 abs / 1e-2 rel); the residual stream
and the V store are bf16 copies/adds and must be bit-exact.  The whole bf16
forward is held to a relative Frobenius error of 2e-2 on the logits, which
any wiring mistake (wrong weight, head order, missing residual, wrong
position) exceeds by orders of magnitude."""

import math

import pytest
import torch
import torch.nn.functional as F

from naivllm_amd.layers import qwen3 as qm
from naivllm_amd.layers.qwen3 import Qwen3Config, Qwen3Verify

pytestmark = pytest.mark.gpu

BF16 = dict(atol=2e-2, rtol=1e-2)


def gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def randn(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g, device="cuda") * scale).to(torch.bfloat16)


@pytest.mark.parametrize("T,E", [(1, 256), (9, 1024), (72, 4096), (5, 1000)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rms_norm(T, E, with_residual):
    print(f"case: rms_norm T={T} E={E} residual={with_residual}", flush=True)
    g = gen(T * 7 + E)
    x, w = randn(g, T, E), randn(g, E)
    res = randn(g, T, E) if with_residual else None
    out = torch.empty_like(x)
    res_out = torch.empty_like(x)
    qm.rms_norm(x, w, 1e-6, out, residual=res, residual_out=res_out)
    r = (x + res) if with_residual else x  # bf16 add: fp32 sum rounded once
    assert torch.equal(res_out, r)
    rf = r.float()
    want = rf / torch.sqrt(rf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    torch.testing.assert_close(out.float(), want, **BF16)


def epilogue_reference(qkv, qw, kw, cos_sin, positions, H, Hkv, D, eps):
    T = qkv.shape[0]
    x = qkv.float().view(T, H + 2 * Hkv, D)
    q, k, v = x[:, :H], x[:, H:H + Hkv], x[:, H + Hkv:]

    def norm(t, w):
        t = t / torch.sqrt(t.pow(2).mean(-1, keepdim=True) + eps) * w.float()
        return t.to(torch.bfloat16).float()  # q_norm / k_norm emit bf16

    cs = cos_sin[positions.clamp(min=0)]
    c, s = cs[:, None, :D // 2], cs[:, None, D // 2:]

    def rope(t):
        t1, t2 = t[..., :D // 2], t[..., D // 2:]
        return torch.cat([t1 * c - t2 * s, t1 * s + t2 * c], -1)

    return rope(norm(q, qw)), rope(norm(k, kw)), v


@pytest.mark.parametrize("D", [64, 128])
def test_qk_norm_rope_store(D):
    print(f"case: qk_norm_rope_store D={D}", flush=True)
    H, Hkv, T, nb, bs = 4, 2, 13, 6, 8
    g = gen(D)
    cfg = Qwen3Config(head_dim=D, max_position=4096)
    cos_sin = qm.rope_cache(cfg, "cuda")
    qkv = randn(g, T, (H + 2 * Hkv) * D, scale=3.0)
    qw, kw = randn(g, D), randn(g, D)
    positions = torch.tensor([0, 1, 7, 100, 4095, 3000, -1, 17, 18, 19, 2, 2047, 9], device="cuda")
    slots = torch.tensor([3, 4, 40, 41, 0, 47, -1, 20, 21, -1, 22, 23, 30], device="cuda")
    q_out = torch.zeros(T, H, D, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros(nb, bs, Hkv, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    qm.qk_norm_rope_store(qkv, qw, kw, cos_sin, positions, slots, q_out, kc, vc, H, Hkv, D, 1e-6)
    wq, wk, wv = epilogue_reference(qkv, qw, kw, cos_sin, positions, H, Hkv, D, 1e-6)
    live = positions >= 0
    torch.testing.assert_close(q_out[live].float(), wq[live], **BF16)
    kflat, vflat = kc.view(nb * bs, Hkv, D), vc.view(nb * bs, Hkv, D)
    stored = slots >= 0
    torch.testing.assert_close(kflat[slots[stored]].float(), wk[stored], **BF16)
    assert torch.equal(vflat[slots[stored]], wv[stored].to(torch.bfloat16))
    untouched = torch.ones(nb * bs, dtype=torch.bool, device="cuda")
    untouched[slots[stored]] = False
    assert not kflat[untouched].any() and not vflat[untouched].any()
    # the rotary table gathered per row (positions None; position -1 takes row 0)
    # gives the same bits as the position lookup
    rows = cos_sin.index_select(0, positions.clamp(0, cos_sin.shape[0] - 1))
    q2, kc2, vc2 = torch.zeros_like(q_out), torch.zeros_like(kc), torch.zeros_like(vc)
    qm.qk_norm_rope_store(qkv, qw, kw, rows, None, slots, q2, kc2, vc2, H, Hkv, D, 1e-6)
    assert torch.equal(q2, q_out) and torch.equal(kc2, kc) and torch.equal(vc2, vc)


@pytest.mark.parametrize("T,E", [(9, 1024), (72, 1024), (3, 4096)])
def test_embed_rms_norm(T, E):
    # the forward's prologue against F.embedding + the fp32 RMSNorm and the
    # rotary cache lookup: the residual stream is the embedding row exactly,
    # the rotary rows are copies; an id past the vocabulary reads row 0 (the
    # reference's single-GPU lookup), a position -1 takes rotary row 0
    print(f"case: embed_rms_norm T={T} E={E}", flush=True)
    g = gen(T + E)
    V, D = 500, 128
    embed, w = randn(g, V, E), randn(g, E)
    ids = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(T)).cuda()
    ids[0] = V + 7
    positions = torch.randint(0, 4096, (T,), generator=torch.Generator().manual_seed(E)).cuda()
    positions[-1] = -1
    cos_sin = qm.rope_cache(Qwen3Config(head_dim=D, max_position=4096), "cuda")
    resid = torch.empty(T, E, dtype=torch.bfloat16, device="cuda")
    h = torch.empty_like(resid)
    rope = torch.empty(T, D, device="cuda")
    qm.embed_rms_norm(ids, embed, w, 1e-6, resid, h, positions, cos_sin, rope)
    x = F.embedding(torch.where(ids < V, ids, torch.zeros_like(ids)), embed)
    assert torch.equal(resid, x)
    xf = x.float()
    want = xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    torch.testing.assert_close(h.float(), want, **BF16)
    assert torch.equal(rope, cos_sin[positions.clamp(0, 4095)])


@pytest.mark.parametrize("T,I", [(1, 512), (72, 3072), (3, 1000)])
def test_silu_mul(T, I):
    print(f"case: silu_mul T={T} I={I}", flush=True)
    g = gen(T + I)
    gu = randn(g, T, 2 * I, scale=4.0)
    out = torch.empty(T, I, dtype=torch.bfloat16, device="cuda")
    qm.silu_mul(gu, out)
    gf, uf = gu.float()[:, :I], gu.float()[:, I:]
    torch.testing.assert_close(out.float(), F.silu(gf) * uf, **BF16)


def dense_forward(model: Qwen3Verify, ids: torch.Tensor) -> torch.Tensor:
    """fp32 causal forward of one sequence (all positions) with the same
    weights, following models/qwen3.py:11-344 op by op."""
    cfg = model.cfg
    H, Hkv, D, E = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden_size
    eps = cfg.rms_norm_eps
    f = lambda t: t.float()  # noqa: E731

    def norm(x, w):
        return x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps) * f(w)

    n = ids.shape[0]
    pos = torch.arange(n, device="cuda")
    cs = model.rope[pos]
    c, s = cs[:, None, :D // 2], cs[:, None, D // 2:]

    def rope(t):
        t1, t2 = t[..., :D // 2], t[..., D // 2:]
        return torch.cat([t1 * c - t2 * s, t1 * s + t2 * c], -1)

    x = f(model.embed)[ids]
    mask = torch.ones(n, n, device="cuda", dtype=torch.bool).tril()
    for L in model.layers:
        h = norm(x, L["ln1"])
        qkv = h @ f(L["qkv"]).t()
        q = qkv[:, :H * D].view(n, H, D)
        k = qkv[:, H * D:(H + Hkv) * D].view(n, Hkv, D)
        v = qkv[:, (H + Hkv) * D:].view(n, Hkv, D)
        q, k = rope(norm(q, L["q_norm"])), rope(norm(k, L["k_norm"]))
        k = k.repeat_interleave(H // Hkv, dim=1)
        v = v.repeat_interleave(H // Hkv, dim=1)
        sc = torch.einsum("qhd,khd->hqk", q, k) / math.sqrt(D)
        sc = sc.masked_fill(~mask, float("-inf"))
        o = torch.einsum("hqk,khd->qhd", sc.softmax(-1), v).reshape(n, H * D)
        x = x + o @ f(L["o"]).t()
        h = norm(x, L["ln2"])
        gu = h @ f(L["gate_up"]).t()
        x = x + (F.silu(gu[:, :cfg.intermediate_size]) * gu[:, cfg.intermediate_size:]) @ f(L["down"]).t()
    return norm(x, model.norm) @ f(model.lm_head).t()


@pytest.mark.parametrize("fused,bs,head_few", [(True, 16, False), (True, 32, True), (False, 16, False)])
def test_forward_matches_dense_fp32(fused, bs, head_few, monkeypatch):
    # two sequences: a first chunk written into a fresh paged cache, then a
    # 9-row verify chunk reading it back, against a dense fp32 forward; both
    # the fused few-row path and the hipBLASLt path of wider batches, 16- and
    # 32-key pages, the LM head on hipBLASLt or on the few-row kernel
    print(f"case: qwen3 verify forward vs dense fp32, fused={fused} block_size={bs} head_few={head_few}", flush=True)
    monkeypatch.setattr(qm, "FUSED_ROWS", 1 << 30 if fused else 0)
    monkeypatch.setattr(qm, "FUSED_ROWS_WIDE", 1 << 30 if fused else 0)
    monkeypatch.setattr(qm, "lm_head_rows", (lambda hidden: 1 << 30) if head_few else (lambda hidden: 0))
    cfg = Qwen3Config(vocab_size=2048, hidden_size=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=64,
                      intermediate_size=512, max_position=4096)
    model = Qwen3Verify(cfg, "cuda", seed=3)
    g = gen(11)
    for L in model.layers:  # non-trivial norm weights, so a swapped weight shows
        for key in ("ln1", "ln2", "q_norm", "k_norm"):
            L[key] = (1.0 + 0.3 * torch.randn(L[key].shape, generator=g, device="cuda")).to(torch.bfloat16)
    model.allocate_kv_cache(16, bs)
    lens1, lens2 = [20, 7], [9, 9]
    seqs = [torch.randint(0, cfg.vocab_size, (a + b,), generator=g, device="cuda") for a, b in zip(lens1, lens2)]
    tables = torch.tensor([[5, 2, 9, -1], [1, 12, -1, -1]], dtype=torch.int32, device="cuda")

    def run(lo, hi):
        ids, pos, slots, cu = [], [], [], [0]
        for b, s in enumerate(seqs):
            p = torch.arange(lo[b], hi[b], device="cuda")
            ids.append(s[lo[b]:hi[b]])
            pos.append(p)
            slots.append(tables[b].long()[p // bs] * bs + p % bs)
            cu.append(cu[-1] + hi[b] - lo[b])
        ctx = torch.tensor(hi, dtype=torch.int64, device="cuda")
        cu_t = torch.tensor(cu, dtype=torch.int32, device="cuda")
        logits = model.forward(torch.cat(ids), torch.cat(pos), torch.cat(slots), tables, ctx, cu_t,
                               max(h - l for l, h in zip(lo, hi)))
        return logits.float().split([h - l for l, h in zip(lo, hi)])

    first = run([0, 0], lens1)
    second = run(lens1, [a + b for a, b in zip(lens1, lens2)])
    for b, s in enumerate(seqs):
        want = dense_forward(model, s)
        got = torch.cat([first[b], second[b]])
        rel = (got - want).norm() / want.norm()
        assert rel < 2e-2, (b, float(rel))

