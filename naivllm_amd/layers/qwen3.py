"""Qwen3 verify forward on the MI355X path.

The target model of the verification round (src/myvllm/models/qwen3.py:
Qwen3Attention :11-123, Qwen3MLP :129-151, Qwen3DecoderLayer :159-227,
Qwen3Model :233-281, Qwen3ForCausalLM :287-344): embedding, N decoder
layers (RMSNorm, fused QKV projection, per-head q/k RMSNorm, NeoX RoPE,
paged KV store + paged verify attention, o_proj, RMSNorm with residual,
SwiGLU MLP), final norm, LM head over every row.  Up to fused_rows() verify
rows every layer runs on this library's gfx950 kernels, 6 launches per
layer: the QKV projection (with the input RMSNorm as its prologue), the
pre-attention epilogue (q/k RMSNorm + RoPE + paged KV store), verify
attention, o_proj (with the residual add as its epilogue), gate_up
(post-attention RMSNorm prologue, SiLU * up epilogue) and down (residual
add epilogue).  Wider batches run the projections on hipBLASLt between
this library's residual-RMSNorm, epilogue, attention and SiLU kernels.  The
LM head runs on this library's streaming kernel up to lm_head_rows() rows
(79 at hidden 1024, 19 at hidden 4096: the activations staged in one CU's
LDS), from a copy of its weight packed in that kernel's load order, and on
hipBLASLt beyond.  Weights are random (seeded): no checkpoint is
loaded.

The forward takes the verify metadata explicitly (positions, slots, block
tables, context lengths, cu_seqlens) so a whole forward is capturable in a
hipGraph with static buffers, as the reference's verify graphs are
(engine/model_runner.py:648-721).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from naivllm_amd import _lib
from naivllm_amd.layers.attention import paged_attention_verify


@dataclass
class Qwen3Config:
    vocab_size: int = 151936
    hidden_size: int = 1024
    num_layers: int = 28
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 3072
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_position: int = 40960
    tie_word_embeddings: bool = True

    @staticmethod
    def qwen3_0_6b(**kw) -> "Qwen3Config":
        return Qwen3Config(**kw)

    @staticmethod
    def qwen3_8b(**kw) -> "Qwen3Config":
        base = dict(hidden_size=4096, num_layers=36, num_heads=32, num_kv_heads=8, head_dim=128,
                    intermediate_size=12288, tie_word_embeddings=False)
        base.update(kw)
        return Qwen3Config(**base)


def rope_cache(cfg: Qwen3Config, device) -> torch.Tensor:
    """[max_position, head_dim] = [cos | sin] of NeoX rotary embedding
    (layers/rotary_embedding.py:48-72), fp32."""
    d = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    pos = torch.arange(cfg.max_position, dtype=torch.float64)
    f = torch.outer(pos, inv)
    return torch.cat([torch.cos(f), torch.sin(f)], dim=-1).float().contiguous().to(device)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor,
             residual: torch.Tensor | None = None, residual_out: torch.Tensor | None = None) -> None:
    """out = rmsnorm(x + residual) * weight; x + residual goes to
    residual_out (layers/layernorm.py:18-35)."""
    T, E = x.shape
    rc = _lib.lib().nsv_rms_norm(x.data_ptr(), _lib.ptr(residual), _lib.ptr(residual_out), weight.data_ptr(),
                                 out.data_ptr(), T, E, eps, _lib.stream_ptr(x.device))
    _lib.check(rc, "rms_norm")


def embed_rms_norm(ids: torch.Tensor, embed: torch.Tensor, weight: torch.Tensor, eps: float, residual_out, out,
                   positions: torch.Tensor | None = None, cos_sin: torch.Tensor | None = None,
                   rope_out: torch.Tensor | None = None) -> None:
    """The forward's prologue (nsv_embed_rms_norm): residual_out = embed[ids],
    out = rmsnorm(residual_out) * weight, and rope_out [T, D] = cos_sin rows
    at the (clamped) positions when given."""
    ids = ids.to(torch.int64).contiguous()
    T, E = residual_out.shape
    D = cos_sin.shape[1] if cos_sin is not None else 0
    rc = _lib.lib().nsv_embed_rms_norm(
        ids.data_ptr(), embed.data_ptr(), embed.shape[0], weight.data_ptr(), eps, residual_out.data_ptr(),
        out.data_ptr(), T, E, _lib.ptr(positions), _lib.ptr(cos_sin), cos_sin.shape[0] if cos_sin is not None else 0,
        D, _lib.ptr(rope_out), _lib.stream_ptr(residual_out.device))
    _lib.check(rc, "embed_rms_norm")


def qk_norm_rope_store(qkv, q_norm_w, k_norm_w, cos_sin, positions, slot_mapping, q_out, k_cache, v_cache,
                       H: int, Hkv: int, D: int, eps: float) -> None:
    """The pre-attention epilogue (nsv_qk_norm_rope_store).  positions None:
    cos_sin holds the rotary row of each step row ([T, D])."""
    rc = _lib.lib().nsv_qk_norm_rope_store(
        qkv.data_ptr(), q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos_sin.data_ptr(), cos_sin.shape[0],
        _lib.ptr(positions), slot_mapping.data_ptr(), q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        qkv.shape[0], H, Hkv, D, eps, _lib.stream_ptr(qkv.device))
    _lib.check(rc, "qk_norm_rope_store")


def decode_fits(hidden: int, attn_dim: int, intermediate: int) -> bool:
    """Whether every projection's reduction suits nsv_linear_decode, and the
    partial sums of the hidden size fit its prologue (at most 256 slots)."""
    return all(k in (1024, 2048, 3072, 4096) for k in (hidden, attn_dim, intermediate)) and hidden // 4 <= 256


def decode_ss_rows(M: int, N: int) -> int:
    """Partial-sum rows a decode-shaped residual epilogue writes (nsv_linear_decode)."""
    return int(_lib.lib().nsv_linear_decode_ss_rows(M, N))


def ss_rows(M: int, N: int, K: int, has_norm: bool = False) -> int:
    """Rows of partial sums of r^2 a residual-epilogue linear writes (one per
    16- or 8-column tile of the output)."""
    return int(_lib.lib().nsv_linear_ss_rows(M, N, K, int(has_norm)))


def lm_head(x: torch.Tensor, packed: torch.Tensor, y: torch.Tensor) -> None:
    """y = x @ W.T (ParallelLMHead.forward's F.linear) from W's copy written
    by nsv_lm_head_pack, on the streaming kernel (nsv_lm_head): the same bits
    as linear(x, W, y)."""
    M, K = x.shape
    N = y.shape[1]
    if (tuple(packed.shape) != (N, K) or y.shape[0] != M or not (x.is_contiguous() and y.is_contiguous())
            or not (x.dtype == packed.dtype == y.dtype == torch.bfloat16)):
        raise ValueError("lm_head: x [M, K], packed [N, K] and y [M, N], contiguous bf16")
    rc = _lib.lib().nsv_lm_head(x.data_ptr(), packed.data_ptr(), y.data_ptr(), M, N, K, _lib.stream_ptr(x.device))
    _lib.check(rc, "lm_head")


def linear(x: torch.Tensor, weight: torch.Tensor, y: torch.Tensor | None = None, *,
           norm_w: torch.Tensor | None = None, ss_in: torch.Tensor | None = None, eps: float = 1e-6,
           swiglu: bool = False, resid: torch.Tensor | None = None, ss_out: torch.Tensor | None = None,
           decode: bool = False) -> None:
    """y = h @ weight.T on this library's few-row kernel (nsv_linear), or,
    decode=True, on its one-wave-per-column kernel for one or two rows
    (nsv_linear_decode: ss_out then has decode_ss_rows(M, N) rows).

    h = rmsnorm(x) * norm_w when norm_w is given (x is then the residual
    stream and ss_in [n, M] the producer's partial sums of x^2), else x.
    swiglu: weight is [gate; up] and y = silu(gate) * up.  resid: instead of
    writing y, add the product into the residual stream resid [M, N] and
    write the new partial sums of resid^2 to ss_out [ss_rows(M, N, K), M]."""
    M, K = x.shape
    N = weight.shape[0]
    epi = 2 if resid is not None else (1 if swiglu else 0)
    nss = ss_in.shape[0] if ss_in is not None else 0
    h = _lib.lib()
    if decode:
        rc = h.nsv_linear_decode(x.data_ptr(), _lib.ptr(norm_w), _lib.ptr(ss_in), nss, eps, weight.data_ptr(),
                                 _lib.ptr(y), _lib.ptr(resid), _lib.ptr(ss_out), M, N, K, epi,
                                 _lib.stream_ptr(x.device))
        _lib.check(rc, "linear_decode")
        return
    nbytes = h.nsv_linear_workspace_size(M, N, K)
    ws = _lib.workspace(x.device, nbytes, "linear")
    rc = h.nsv_linear(x.data_ptr(), _lib.ptr(norm_w), _lib.ptr(ss_in), nss, eps, weight.data_ptr(),
                      _lib.ptr(y), _lib.ptr(resid), _lib.ptr(ss_out), M, N, K, epi, _lib.ptr(ws),
                      ws.numel() if ws is not None else 0, _lib.stream_ptr(x.device))
    _lib.check(rc, "linear")


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor) -> None:
    rc = _lib.lib().nsv_silu_mul(gate_up.data_ptr(), out.data_ptr(), gate_up.shape[0], out.shape[1],
                                 _lib.stream_ptr(gate_up.device))
    _lib.check(rc, "silu_mul")


# Verify rows up to which the forward runs on the fused few-row linear
# kernel.  Every workgroup of that kernel reads the whole activation block,
# so its cost grows with rows x hidden size, while hipBLASLt's wide tiles
# reuse the activations.  Measured on MI355X (each projection alone): at
# hidden 1024 the fused layer (4 launches) beats hipBLASLt + the separate
# norm / SiLU kernels up to 72 rows (38 vs 42 us per layer at 72); at hidden
# 4096 the fused kernel wins at 9 rows and loses from about 16.
FUSED_ROWS = 80
FUSED_ROWS_WIDE = 12  # hidden size above 2048


# Rows up to which the LM head runs on this library's kernels: nsv_linear
# streams a vocabulary-wide head's weight tiles while the activations fit its
# LDS (rows x (hidden + 8) bf16 within 160 KiB), hipBLASLt's large tiles
# beyond.  Measured on MI355X, graph-replayed, the 0.6B head alone: 58.6 vs
# 58.6 us at 9 rows, 59.9 vs 69.2 at 18, 70.5 vs 83.7 at 72; the 8B head
# (hidden 4096): 232 vs 248 us at 9 rows.
LM_HEAD_LDS = 160 * 1024


def lm_head_rows(hidden: int) -> int:
    return max(16, min(79, LM_HEAD_LDS // ((hidden + 8) * 2)))


def prefill_metadata(token_lists, starts, tables, block_size: int, q_block: int, device):
    """Rows of one prefill forward over several sequences' new tokens.

    Sequence i contributes its tokens starts[i] .. len(token_lists[i]) - 1 at
    their positions (the pages before starts[i] already hold their KV: a
    cached prefix).  Its rows are cut into causal blocks of q_block rows;
    each block is one entry of the verify attention's batch, whose context
    ends at the block's last position and whose block-table row is the
    sequence's, so every row attends exactly the keys 0 .. its position.
    Returns (input_ids, positions, slot_mapping, block_tables, context_lens,
    cu_seqlens_q, last_rows) on ``device``; last_rows[i] is the row of
    sequence i's last token."""
    import numpy as np

    ids, pos, slots, ctx, cu, bt_rows, last = [], [], [], [], [0], [], []
    width = max(len(t) for t in tables)
    for toks, start, table in zip(token_lists, starts, tables):
        n = len(toks)
        if not 0 <= start < n:
            raise ValueError(f"prefill start {start} outside a {n}-token sequence")
        p = np.arange(start, n, dtype=np.int64)
        page = np.asarray(table, dtype=np.int64)[p // block_size]
        ids.append(np.asarray(toks[start:], dtype=np.int64))
        pos.append(p)
        slots.append(page * block_size + p % block_size)
        row = np.full(width, -1, dtype=np.int32)
        row[:len(table)] = table
        for b0 in range(start, n, q_block):
            b1 = min(n, b0 + q_block)
            ctx.append(b1)
            cu.append(cu[-1] + (b1 - b0))
            bt_rows.append(row)
        last.append(cu[-1] - 1)
    t = lambda x, dt: torch.from_numpy(np.ascontiguousarray(x, dtype=dt)).to(device)  # noqa: E731
    return (t(np.concatenate(ids), np.int64), t(np.concatenate(pos), np.int64), t(np.concatenate(slots), np.int64),
            t(np.stack(bt_rows), np.int32), t(ctx, np.int64), t(cu, np.int32), t(last, np.int64))


def fused_rows(hidden_size: int) -> int:
    return FUSED_ROWS if hidden_size <= 2048 else FUSED_ROWS_WIDE


class Qwen3Verify:
    """Random-init Qwen3 weights plus the verify forward."""

    def __init__(self, cfg: Qwen3Config, device, dtype=torch.bfloat16, seed: int = 0, std: float = 0.02):
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = dtype
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)

        def w(*shape, scale=std):
            return (torch.randn(*shape, generator=g, device=self.device, dtype=torch.float32) * scale).to(dtype)

        H, Hkv, D, E = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden_size
        self.embed = w(cfg.vocab_size, E, scale=1.0)
        self.layers = []
        for _ in range(cfg.num_layers):
            self.layers.append(dict(
                ln1=torch.ones(E, device=self.device, dtype=dtype),
                qkv=w((H + 2 * Hkv) * D, E, scale=1.0 / math.sqrt(E)),
                q_norm=torch.ones(D, device=self.device, dtype=dtype),
                k_norm=torch.ones(D, device=self.device, dtype=dtype),
                o=w(E, H * D, scale=1.0 / math.sqrt(H * D)),
                ln2=torch.ones(E, device=self.device, dtype=dtype),
                gate_up=w(2 * cfg.intermediate_size, E, scale=1.0 / math.sqrt(E)),
                down=w(E, cfg.intermediate_size, scale=1.0 / math.sqrt(cfg.intermediate_size)),
            ))
        self.norm = torch.ones(E, device=self.device, dtype=dtype)
        self.lm_head = self.embed if cfg.tie_word_embeddings else w(cfg.vocab_size, E, scale=1.0 / math.sqrt(E))
        self.pack_lm_head()
        self.rope = rope_cache(cfg, self.device)
        self.scale = 1.0 / math.sqrt(D)
        self.k_caches: list[torch.Tensor] = []
        self.v_caches: list[torch.Tensor] = []
        self.block_size = 0
        # forwards of one or two rows take the one-wave-per-column projections
        # (a drafter's steps; the target keeps one kernel family at every row
        # count, so its rows come out the same at every batch shape)
        self.decode_linears = False


    def pack_lm_head(self) -> None:
        """Repack the LM head's weight in the streaming kernel's load order
        (nsv_lm_head_pack) where this shape streams; the row-major weight
        stays for the embedding lookup and for more rows than that.  Called
        once by the constructor; whoever replaces or edits self.lm_head
        afterwards calls it again."""
        self.lm_head_packed = None
        self.lm_head_packed_rows = 0
        if self.device.type != "cuda" or self.lm_head.dtype != torch.bfloat16:
            return
        V, E = self.lm_head.shape
        self.lm_head_packed_rows = _lib.lib().nsv_lm_head_rows(V, E)
        if self.lm_head_packed_rows > 0:
            self.lm_head_packed = torch.empty_like(self.lm_head)
            _lib.check(_lib.lib().nsv_lm_head_pack(self.lm_head.data_ptr(), self.lm_head_packed.data_ptr(), V, E,
                                                   _lib.stream_ptr(self.device)), "lm_head_pack")
    def prefill_q_block(self) -> int:
        """Query rows per causal block of a prefill: the verify kernel serves
        up to 64 (GQA group x rows) per (sequence, kv head)."""
        return 64 // (self.cfg.num_heads // self.cfg.num_kv_heads)

    @torch.inference_mode()
    def prefill(self, token_lists, starts, tables) -> torch.Tensor:
        """One forward over the new tokens of several sequences (see
        prefill_metadata): their K/V land in the paged cache, and the logits
        of each sequence's last token come back, [len(token_lists), vocab]."""
        ids, pos, slots, bt, ctx, cu, last = prefill_metadata(token_lists, starts, tables, self.block_size,
                                                              self.prefill_q_block(), self.device)
        return self.forward(ids, pos, slots, bt, ctx, cu, self.prefill_q_block(), logits_rows=last)

    def allocate_kv_cache(self, num_blocks: int, block_size: int) -> None:
        """One [num_blocks, block_size, Hkv, D] K and V pool per layer
        (engine/model_runner.py:244-279 keeps one [2, L, ...] tensor)."""
        cfg = self.cfg
        shape = (num_blocks, block_size, cfg.num_kv_heads, cfg.head_dim)
        self.k_caches = [torch.zeros(shape, device=self.device, dtype=self.dtype) for _ in range(cfg.num_layers)]
        self.v_caches = [torch.zeros(shape, device=self.device, dtype=self.dtype) for _ in range(cfg.num_layers)]
        self.block_size = block_size

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, slot_mapping: torch.Tensor,
                block_tables: torch.Tensor, context_lens: torch.Tensor, cu_seqlens_q: torch.Tensor,
                max_q_len: int, logits_out: torch.Tensor | None = None,
                logits_rows: torch.Tensor | None = None) -> torch.Tensor:
        """Verify forward over T = sum of per-sequence query rows.  Rows at
        position -1 are inert padding (no KV store, zero attention output).
        Returns logits [T, vocab] (written into logits_out when given), or
        only the rows ``logits_rows`` indexes (the prefill's last rows)."""
        if self.dtype != torch.bfloat16:
            raise ValueError("the fused forward kernels are bf16")
        cfg = self.cfg
        H, Hkv, D, E = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden_size
        eps = cfg.rms_norm_eps
        T = input_ids.shape[0]
        block_m = max(16, 1 << (max_q_len - 1).bit_length())
        I = cfg.intermediate_size
        resid = torch.empty(T, E, dtype=self.dtype, device=self.device)  # the residual stream
        h = torch.empty_like(resid)
        q = torch.empty(T, H, D, dtype=self.dtype, device=self.device)
        attn = lambda li: paged_attention_verify(  # noqa: E731
            q, self.k_caches[li], self.v_caches[li], block_tables, context_lens, cu_seqlens_q, positions,
            self.scale, H, Hkv, D, self.block_size, block_m, max_q_len=max_q_len)
        # embedding lookup, layer 0's input norm, and the rotary rows of the step's
        # positions (gathered once for every layer, so that each layer's epilogue
        # loads them without first loading the positions) in one launch
        rope_rows = torch.empty(T, D, dtype=torch.float32, device=self.device)
        embed_rms_norm(input_ids, self.embed, self.layers[0]["ln1"], eps, resid, h, positions, self.rope, rope_rows)
        if T <= fused_rows(E):
            # Every RMSNorm after layer 0's is the prologue of the projection
            # that consumes it and every residual add the epilogue of the
            # projection that produces it: 6 launches per layer.
            qkv = torch.empty(T, (H + 2 * Hkv) * D, dtype=self.dtype, device=self.device)
            act = torch.empty(T, I, dtype=self.dtype, device=self.device)
            # one or two rows on a drafter: the one-wave-per-column kernel
            dec = self.decode_linears and T <= 2 and decode_fits(E, H * D, I)
            # partial sums of resid^2 from o_proj and down (their tiles' count)
            ss_o = torch.empty(decode_ss_rows(T, E) if dec else ss_rows(T, E, H * D), T, dtype=torch.float32,
                               device=self.device)
            ss_d = torch.empty(decode_ss_rows(T, E) if dec else ss_rows(T, E, I), T, dtype=torch.float32,
                               device=self.device)
            for li, L in enumerate(self.layers):
                if li == 0:
                    linear(h, L["qkv"], qkv, decode=dec)
                else:
                    linear(resid, L["qkv"], qkv, norm_w=L["ln1"], ss_in=ss_d, eps=eps, decode=dec)
                qk_norm_rope_store(qkv, L["q_norm"], L["k_norm"], rope_rows, None, slot_mapping, q,
                                   self.k_caches[li], self.v_caches[li], H, Hkv, D, eps)
                linear(attn(li).view(T, H * D), L["o"], resid=resid, ss_out=ss_o, decode=dec)
                linear(resid, L["gate_up"], act, norm_w=L["ln2"], ss_in=ss_o, eps=eps, swiglu=True, decode=dec)
                linear(act, L["down"], resid=resid, ss_out=ss_d, decode=dec)
            rms_norm(resid, self.norm, eps, h)
        else:
            # wider batches: hipBLASLt projections between this library's
            # norm / epilogue / SiLU kernels (9 launches per layer)
            act = torch.empty(T, I, dtype=self.dtype, device=self.device)
            for li, L in enumerate(self.layers):
                if li > 0:
                    rms_norm(x, L["ln1"], eps, h, residual=resid, residual_out=resid)
                qkv = F.linear(h, L["qkv"])
                qk_norm_rope_store(qkv, L["q_norm"], L["k_norm"], rope_rows, None, slot_mapping, q,
                                   self.k_caches[li], self.v_caches[li], H, Hkv, D, eps)
                x = F.linear(attn(li).view(T, H * D), L["o"])
                rms_norm(x, L["ln2"], eps, h, residual=resid, residual_out=resid)
                silu_mul(F.linear(h, L["gate_up"]), act)
                x = F.linear(act, L["down"])
            rms_norm(x, self.norm, eps, h, residual=resid)
        if logits_rows is not None:
            h = h.index_select(0, logits_rows)
            T = h.shape[0]
        # the LM head: this library's streaming kernel up to lm_head_rows rows
        # (it streams the vocabulary's weight rows faster there), hipBLASLt's
        # large tiles beyond
        if T <= lm_head_rows(E):
            if logits_out is None:
                logits_out = torch.empty(T, self.lm_head.shape[0], dtype=self.dtype, device=self.device)
            if self.lm_head_packed is not None and T <= self.lm_head_packed_rows:
                lm_head(h, self.lm_head_packed, logits_out)
            else:
                linear(h, self.lm_head, logits_out)
            return logits_out
        if logits_out is None:
            return F.linear(h, self.lm_head)
        torch.matmul(h, self.lm_head.t(), out=logits_out)
        return logits_out
