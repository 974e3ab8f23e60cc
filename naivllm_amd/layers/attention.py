"""Verify-attention and KV-store operators with the reference's signatures.

Drop-in for ``paged_attention_verify`` and ``store_kvcache`` of
src/myvllm/layers/attention.py (:615-668 and :71-112) and for the verify
branch of ``Attention.forward`` (:689-731).  Both operators launch the
gfx950 kernels of libnaivspec.so on torch's current stream; there is no
PyTorch fallback.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from naivllm_amd import _lib
from naivllm_amd.utils.context import get_context

_INDEX_DTYPES = {
    "block_tables": torch.int32,
    "context_lens": torch.int64,
    "cu_seqlens_q": torch.int32,
    "positions": torch.int64,
    "slot_mapping": torch.int64,
}


def _as(t: torch.Tensor, name: str) -> torch.Tensor:
    want = _INDEX_DTYPES[name]
    if t.dtype != want:
        t = t.to(want)
    return t if t.is_contiguous() else t.contiguous()


def _check_cache(cache: torch.Tensor, name: str) -> tuple[int, int, int, int]:
    if cache.dim() != 4:
        raise ValueError(f"{name} must be (num_blocks, block_size, num_kv_heads, head_dim), got {tuple(cache.shape)}")
    if not cache.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return tuple(cache.shape)


def verify_attention_workspace_bytes(batch_size: int, num_heads: int, num_kv_heads: int, head_dim: int,
                                     block_size: int, max_num_blocks: int, max_q_len: int,
                                     dtype: torch.dtype, kv_split_tokens: int = 0) -> int:
    return int(_lib.lib().nsv_verify_attention_workspace_size(
        batch_size, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks, max_q_len,
        _lib.dtype_code(dtype), kv_split_tokens))


ATTN_KERNELS = {0: "d-sliced", 1: "key-split", 2: "fp32"}


def verify_attention_plan(batch_size: int, num_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                          max_num_blocks: int, max_q_len: int, dtype: torch.dtype, kv_split_tokens: int = 0,
                          cus: int = 0) -> tuple[str, int]:
    """(kernel, key splits per sequence) that paged_attention_verify runs for
    this shape on a device with ``cus`` compute units (0: the current one)."""
    import ctypes
    kind, splits = ctypes.c_int(), ctypes.c_int()
    rc = _lib.lib().nsv_verify_attention_plan(batch_size, num_heads, num_kv_heads, head_dim, block_size,
                                             max_num_blocks, max_q_len, _lib.dtype_code(dtype), kv_split_tokens,
                                             cus, ctypes.addressof(kind), ctypes.addressof(splits))
    _lib.check(rc, "verify_attention_plan")
    return ATTN_KERNELS[kind.value], splits.value


def paged_attention_verify(
    query: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    positions: torch.Tensor,
    scale: float,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    block_m: int,
    *,
    max_q_len: int | None = None,
    kv_split_tokens: int = 0,
    out: torch.Tensor | None = None,
    allocation_free: bool = False,
) -> torch.Tensor:
    """Verify a chunk of drafted tokens against the paged KV cache.

    Same arguments and result as the reference (layers/attention.py:615-668):
      query (T, H, D); k_cache/v_cache (num_blocks, block_size, Hkv, D);
      block_tables (B, max_num_blocks), -1 padded; context_lens (B,);
      cu_seqlens_q (B+1,); positions (T,), -1 marks an inert pad row;
      block_m >= every per-sequence query length.
    Returns (T, H, D) in query's dtype.  Keyword-only extras: ``max_q_len``
    (a tighter bound than block_m: fewer padded MFMA rows and partials),
    ``kv_split_tokens`` (keys per workgroup split, 0 = automatic), ``out``
    (a preallocated result) and ``allocation_free`` (run through
    nsv_verify_attention_noalloc: the library's fixed per-device scratch
    instead of a workspace, ``out`` required, index tensors already int32 /
    int64 and contiguous, so the call allocates nothing).  Rows at position
    -1 come back as zeros (the reference leaves them meaningless; nothing
    reads them).
    """
    if query.dim() != 3 or query.shape[1] != num_heads or query.shape[2] != head_dim:
        raise ValueError(f"query must be (T, {num_heads}, {head_dim}), got {tuple(query.shape)}")
    nb, bs, hkv, d = _check_cache(k_cache, "k_cache")
    if tuple(v_cache.shape) != (nb, bs, hkv, d) or not v_cache.is_contiguous():
        raise ValueError("k_cache and v_cache must have the same contiguous shape")
    if bs != block_size or hkv != num_kv_heads or d != head_dim:
        raise ValueError("cache shape disagrees with block_size / num_kv_heads / head_dim")
    if query.dtype != k_cache.dtype or v_cache.dtype != k_cache.dtype:
        raise ValueError("query and caches must share one dtype")
    if not query.is_cuda:
        raise ValueError("paged_attention_verify runs on the GPU; query is on the CPU")
    query = query.contiguous()
    block_tables = _as(block_tables, "block_tables")
    context_lens = _as(context_lens, "context_lens")
    cu_seqlens_q = _as(cu_seqlens_q, "cu_seqlens_q")
    positions = _as(positions, "positions")
    batch_size, max_num_blocks = block_tables.shape
    qlen_bound = int(max_q_len if max_q_len is not None else block_m)
    code = _lib.dtype_code(query.dtype)
    h = _lib.lib()
    if out is not None and (tuple(out.shape) != tuple(query.shape) or out.dtype != query.dtype
                            or out.device != query.device or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous {query.dtype} tensor of shape {tuple(query.shape)} on "
                         f"{query.device}")
    if allocation_free:
        if out is None:
            raise ValueError("allocation_free=True needs a preallocated out")
        rc = h.nsv_verify_attention_noalloc(
            out.data_ptr(), query.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_tables.data_ptr(),
            context_lens.data_ptr(), cu_seqlens_q.data_ptr(), positions.data_ptr(), float(scale), batch_size,
            query.shape[0], num_heads, num_kv_heads, head_dim, block_size, max_num_blocks, qlen_bound, code,
            kv_split_tokens, _lib.stream_ptr(query.device))
        _lib.check(rc, "paged_attention_verify (allocation-free)")
        return out
    if out is None:
        out = torch.empty_like(query)
    ws_bytes = int(h.nsv_verify_attention_workspace_size(
        batch_size, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks, qlen_bound, code,
        kv_split_tokens))
    ws = _lib.workspace(query.device, ws_bytes, "verify_attention")
    rc = h.nsv_verify_attention(
        out.data_ptr(), query.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        block_tables.data_ptr(), context_lens.data_ptr(), cu_seqlens_q.data_ptr(), positions.data_ptr(),
        float(scale), batch_size, query.shape[0], num_heads, num_kv_heads, head_dim, block_size,
        max_num_blocks, qlen_bound, code, kv_split_tokens,
        _lib.ptr(ws), ws_bytes, _lib.stream_ptr(query.device))
    _lib.check(rc, "paged_attention_verify")
    return out


def store_kvcache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    block_size: int,
) -> None:
    """Scatter (T, Hkv, D) key/value rows into the paged caches at
    ``slot_mapping`` (slot -1 = skip), as layers/attention.py:71-112."""
    num_tokens, num_kv_heads, head_dim = key.shape
    key = key.contiguous()
    value = value.contiguous()
    if k_cache.shape != v_cache.shape:
        raise ValueError("K and V cache shapes must match")
    if slot_mapping.numel() != num_tokens:
        raise ValueError("Slot mapping size must match number of tokens")
    nb, bs, hkv, d = _check_cache(k_cache, "k_cache")
    if not v_cache.is_contiguous():
        raise ValueError("v_cache must be contiguous")
    if (bs, hkv, d) != (block_size, num_kv_heads, head_dim):
        raise ValueError("cache shape disagrees with key shape / block_size")
    if key.dtype != k_cache.dtype or value.dtype != v_cache.dtype:
        raise ValueError("key/value and caches must share one dtype")
    slot_mapping = _as(slot_mapping, "slot_mapping")
    rc = _lib.lib().nsv_store_kv(
        key.data_ptr(), value.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(),
        num_tokens, num_kv_heads, head_dim, block_size, _lib.dtype_code(key.dtype),
        _lib.stream_ptr(key.device))
    _lib.check(rc, "store_kvcache")


_prefill_plan: tuple = (None, None)  # (the Context it was built for, its tensors)


def _prefill_rows(ctx, num_heads: int, num_kv_heads: int, device) -> tuple:
    """Verify-kernel metadata of a prefill step, built once per Context.

    Sequence i has seqlens_q[i] new rows at positions seqlens_k[i] -
    seqlens_q[i] .. seqlens_k[i] - 1.  Its rows are cut into causal blocks of
    q_block = 64 // G rows (G query heads per kv head: the kernel holds up to
    64 query rows per (sequence, kv head)); each block is one entry of the
    kernel's batch with context = the block's last position + 1, so every
    row attends exactly keys 0 .. its position.  Block-table row of block j:
    the sequence's row of context.block_tables (paged prefill) or, without
    block tables, the sequence's keys in the step's own contiguous K/V read
    as one-token pages (cu_seqlens_k[i] + p for position p).
    Returns (block_tables, context_lens, cu_seqlens_q, positions, q_block)."""
    import numpy as np

    global _prefill_plan
    if _prefill_plan[0] is ctx:
        return _prefill_plan[1]
    if ctx.seqlens_q is None or ctx.seqlens_k is None:
        raise ValueError("a prefill step needs context.seqlens_q and context.seqlens_k")
    q_block = max(1, 64 // (num_heads // num_kv_heads))
    paged = ctx.block_tables is not None
    tables = ctx.block_tables.cpu().numpy() if paged else None
    width = tables.shape[1] if paged else max(ctx.seqlens_k)
    bt, lens, cu, pos = [], [], [0], []
    k_start = 0
    for i, (ql, kl) in enumerate(zip(ctx.seqlens_q, ctx.seqlens_k)):
        if not 0 < ql <= kl:
            raise ValueError(f"prefill sequence {i}: {ql} query rows over {kl} keys")
        if paged:
            row = tables[i].astype(np.int32)
        else:
            row = np.full(width, -1, dtype=np.int32)
            row[:kl] = np.arange(k_start, k_start + kl, dtype=np.int32)
        for b0 in range(kl - ql, kl, q_block):
            b1 = min(kl, b0 + q_block)
            bt.append(row)
            lens.append(b1)
            cu.append(cu[-1] + (b1 - b0))
        pos.append(np.arange(kl - ql, kl, dtype=np.int64))
        k_start += kl
    t = lambda x, dt: torch.from_numpy(np.ascontiguousarray(x, dtype=dt)).to(device)  # noqa: E731
    out = (t(np.stack(bt), np.int32), t(lens, np.int64), t(cu, np.int32), t(np.concatenate(pos), np.int64), q_block)
    _prefill_plan = (ctx, out)
    return out


class Attention(nn.Module):
    """Attention layer of the reference (layers/attention.py:670-767):
    writes this step's K/V into the paged cache at context.slot_mapping,
    then attends from the query rows the global Context describes:
      * verify (context.is_verify): a chunk of drafted tokens per sequence
        with a causal mask from absolute positions (:704-731);
      * prefill (context.is_prefill, :733-757): every new prompt row of each
        sequence, causally over its keys.  With context.block_tables (a
        prompt behind a cached prefix) the keys come from the paged cache,
        the step's own K/V already stored in it, as the reference's
        paged_attention_prefill (:328-363); without, from the step's
        contiguous K/V, as its varlen flash path (:257-325).  Both run on the
        verify kernel over causal blocks of rows (``_prefill_rows``);
      * decode (neither flag): one query row per sequence attending its
        whole context (:759-767), served by the same verify kernel with
        each row at position context_lens - 1."""

    def __init__(self, num_heads: int, head_dim: int, scale: float = 1.0, num_kv_heads: int | None = None,
                 block_size: int = 16):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads if num_kv_heads is not None else num_heads
        self.block_size = block_size
        self.k_cache = self.v_cache = torch.tensor([])

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        context = get_context()
        k_cache, v_cache = self.k_cache, self.v_cache
        if k_cache.numel() > 0 and v_cache.numel() > 0 and context.slot_mapping is not None:
            store_kvcache(k.reshape(-1, self.num_kv_heads, self.head_dim),
                          v.reshape(-1, self.num_kv_heads, self.head_dim),
                          k_cache, v_cache, context.slot_mapping, self.block_size)
        scale = self.scale / (self.head_dim ** 0.5)
        q = q.reshape(-1, self.num_heads, self.head_dim)
        if context.is_prefill and not context.is_verify:
            if context.cu_seqlens_q is None:
                raise ValueError("cu_seqlens_q must be provided for varlen attention")
            bt, lens, cu, positions, q_block = _prefill_rows(context, self.num_heads, self.num_kv_heads, q.device)
            if context.block_tables is not None:
                kc, vc, bs = k_cache, v_cache, self.block_size
            else:  # the step's own keys, one token per page
                kc = k.reshape(-1, 1, self.num_kv_heads, self.head_dim).contiguous()
                vc = v.reshape(-1, 1, self.num_kv_heads, self.head_dim).contiguous()
                bs = 1
            o = paged_attention_verify(q, kc, vc, bt, lens, cu, positions, scale, self.num_heads, self.num_kv_heads,
                                       self.head_dim, bs, max(16, q_block), max_q_len=q_block)
            return o.reshape(o.shape[0], self.num_heads * self.head_dim)
        if context.is_verify:
            max_q_len = max(context.seqlens_q)
            cu, positions = context.cu_seqlens_q, context.positions
        else:
            # decode: row b is the newest token of sequence b
            max_q_len = 1
            cu = torch.arange(0, q.shape[0] + 1, dtype=torch.int32, device=q.device)
            positions = context.context_lens.to(torch.int64) - 1
        block_m = max(16, 1 << (max_q_len - 1).bit_length())
        o = paged_attention_verify(
            q, k_cache, v_cache, context.block_tables, context.context_lens, cu, positions, scale,
            self.num_heads, self.num_kv_heads, self.head_dim, self.block_size, block_m, max_q_len=max_q_len)
        return o.reshape(o.shape[0], self.num_heads * self.head_dim)
