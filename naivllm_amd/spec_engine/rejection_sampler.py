"""Acceptance of drafted tokens, on the GPU.

``RejectionSampler`` keeps the reference's interface
(src/myvllm/spec_engine/rejection_sampler.py:24-98): ``verify_greedy``,
``verify_stochastic`` and ``verify`` take one sequence's drafts and logits
rows and return its accepted tokens.  ``accept_greedy`` /
``accept_stochastic`` are the batched forms the verification round uses:
one launch sequence for every sequence of the round, results left on the
device (no host sync).

Randomness: the reference draws ``torch.rand(K)`` and then one
``torch.multinomial`` (model drafts) or one row-wise multinomial over K+1
rows (n-gram drafts) from ``generator``.  torch's multinomial(p, 1) is
argmax(p / q) with q = empty_like(p).exponential_(1) drawn from the same
generator, so ``draw_randomness`` draws u and q in exactly that order and
the kernels reproduce the reference's samples from them.
"""

from __future__ import annotations

import torch

from naivllm_amd import _lib

GREEDY_TEMPERATURE = 1e-6  # temperature <= this selects greedy (rejection_sampler.py:95)


def _i32(x, device) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x.to(device=device, dtype=torch.int32).contiguous()
    return torch.tensor(x, dtype=torch.int32, device=device)


def _check_logits(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be on the GPU")
    if t.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"{name}: unsupported dtype {t.dtype}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name}: rows must be contiguous")


def _check_extent(t: torch.Tensor, elems: int, name: str) -> None:
    """The kernels address rows from t's first element by strides; make
    sure every addressed element lies inside t's storage."""
    avail = t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()
    if elems > avail:
        raise ValueError(f"{name}: the strides address {elems} elements, the tensor holds {avail}")


def _pad_drafts(draft_lists, K: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    B = len(draft_lists)
    drafts = torch.zeros(B, K, dtype=torch.int32)
    for b, d in enumerate(draft_lists):
        if d:
            drafts[b, :len(d)] = torch.as_tensor(d, dtype=torch.int32)
    nd = torch.tensor([len(d) for d in draft_lists], dtype=torch.int32)
    return drafts.to(device, non_blocking=True), nd.to(device, non_blocking=True)


def accept_greedy(target_logits: torch.Tensor, drafts: torch.Tensor, num_drafts: torch.Tensor,
                  seq_stride: int, out_tokens: torch.Tensor | None = None,
                  out_len: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Batched greedy acceptance.  target_logits [rows, V]: the rows of
    sequence b start at b * seq_stride; drafts [B, K] int32, num_drafts [B].
    Returns (tokens [B, K+1] int32, lengths [B] int32) on the device."""
    _check_logits(target_logits, "target_logits")
    V = target_logits.shape[-1]
    B, K = drafts.shape
    if seq_stride < K + 1:
        raise ValueError("seq_stride must be at least K + 1 rows")
    _check_extent(target_logits, ((B - 1) * seq_stride + K + 1) * V, "target_logits")
    dev = target_logits.device
    drafts = _i32(drafts, dev)
    num_drafts = _i32(num_drafts, dev)
    if out_tokens is None:
        out_tokens = torch.empty(B, K + 1, dtype=torch.int32, device=dev)
    if out_len is None:
        out_len = torch.empty(B, dtype=torch.int32, device=dev)
    h = _lib.lib()
    code = _lib.dtype_code(target_logits.dtype)
    nbytes = int(h.nsv_accept_workspace_size(B, K, V, code, 0))
    ws = _lib.workspace(dev, nbytes, "accept")
    rc = h.nsv_accept_greedy(target_logits.data_ptr(), seq_stride, drafts.data_ptr(), num_drafts.data_ptr(), B, K,
                             V, code, out_tokens.data_ptr(), out_len.data_ptr(), _lib.ptr(ws), nbytes,
                             _lib.stream_ptr(dev))
    _lib.check(rc, "accept_greedy")
    return out_tokens, out_len


def accept_stochastic(target_logits: torch.Tensor, drafts: torch.Tensor, num_drafts: torch.Tensor,
                      temperature: torch.Tensor, noise: torch.Tensor, uniforms: torch.Tensor | None = None,
                      draft_logits: torch.Tensor | None = None, target_seq_stride: int | None = None,
                      draft_seq_stride: int = 0, draft_row_stride: int = 1,
                      draft_mode: torch.Tensor | None = None,
                      out_tokens: torch.Tensor | None = None,
                      out_len: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Batched stochastic acceptance (greedy for sequences whose
    temperature <= 1e-6).  draft_logits None: n-gram mode, noise
    [B, K+1, V]; else model mode: draft row i of sequence b is row
    b*draft_seq_stride + i*draft_row_stride of draft_logits, uniforms
    [B, K] fp32, noise [B, V].  draft_mode [B] int32 (with draft_logits)
    mixes the modes per sequence (0 = n-gram), with noise [B, K+1, V]
    whose row 0 is a model-mode sequence's one multinomial.  noise has the
    logits dtype."""
    _check_logits(target_logits, "target_logits")
    dev = target_logits.device
    V = target_logits.shape[-1]
    B, K = drafts.shape
    if target_seq_stride is None:
        target_seq_stride = K + 1
    if K == 0 and draft_logits is not None:
        # no drafts: the only draw is the bonus multinomial of row 0, the same
        # in both modes ([V] noise == [1, V] noise)
        draft_logits, uniforms = None, None
    if target_seq_stride < K + 1:
        raise ValueError("target_seq_stride must be at least K + 1 rows")
    _check_extent(target_logits, ((B - 1) * target_seq_stride + K + 1) * V, "target_logits")
    if draft_logits is not None:
        _check_logits(draft_logits, "draft_logits")
        if draft_logits.dtype != target_logits.dtype:
            raise ValueError("draft and target logits must share one dtype")
        if draft_row_stride < 1 or draft_seq_stride < 0:
            raise ValueError("bad draft strides")
        if K > 0:
            _check_extent(draft_logits, ((B - 1) * draft_seq_stride + (K - 1) * draft_row_stride + 1) * V,
                          "draft_logits")
        if uniforms is None or uniforms.numel() != B * K:
            raise ValueError("model-draft acceptance needs uniforms of shape (B, K)")
        uniforms = uniforms.to(device=dev, dtype=torch.float32).contiguous()
    if noise.dtype != target_logits.dtype or not noise.is_contiguous():
        raise ValueError("noise must be contiguous and have the logits dtype")
    if draft_mode is not None:
        if draft_logits is None:
            raise ValueError("draft_mode selects per-sequence draft rows; draft_logits is missing")
        draft_mode = _i32(draft_mode, dev)
        if draft_mode.numel() != B:
            raise ValueError("draft_mode must hold one flag per sequence")
    per_seq = V if (draft_logits is not None and draft_mode is None) else (K + 1) * V
    if noise.numel() != B * per_seq:
        raise ValueError(f"noise holds {noise.numel()} values, expected {B * per_seq}")
    drafts = _i32(drafts, dev)
    num_drafts = _i32(num_drafts, dev)
    temperature = temperature.to(device=dev, dtype=torch.float32).contiguous()
    if out_tokens is None:
        out_tokens = torch.empty(B, K + 1, dtype=torch.int32, device=dev)
    if out_len is None:
        out_len = torch.empty(B, dtype=torch.int32, device=dev)
    h = _lib.lib()
    code = _lib.dtype_code(target_logits.dtype)
    nbytes = int(h.nsv_accept_workspace_size(B, K, V, code, 1))
    ws = _lib.workspace(dev, nbytes, "accept")
    rc = h.nsv_accept_stochastic(
        target_logits.data_ptr(), target_seq_stride, _lib.ptr(draft_logits), draft_seq_stride, draft_row_stride,
        _lib.ptr(draft_mode), drafts.data_ptr(), num_drafts.data_ptr(), temperature.data_ptr(), _lib.ptr(uniforms),
        noise.data_ptr(), per_seq, B, K, V, code, out_tokens.data_ptr(), out_len.data_ptr(), _lib.ptr(ws), nbytes,
        _lib.stream_ptr(dev))
    _lib.check(rc, "accept_stochastic")
    return out_tokens, out_len


def sample(logits: torch.Tensor, temperature: torch.Tensor, noise: torch.Tensor,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """The decode sampler of src/myvllm/layers/sampler.py:14-24 on the
    GPU: logits [B, V] (rows contiguous, any row pitch that is a multiple
    of V), temperature [B] fp32 (<= 1e-6: argmax), noise [B, V] fp32
    exponential draws clamped at 1e-10.  Returns / writes int32 tokens
    [B] (``out`` may be a strided column of a draft buffer)."""
    _check_logits(logits, "logits")
    if logits.dim() != 2:
        raise ValueError("logits must be (batch, vocab)")
    B, V = logits.shape
    dev = logits.device
    if B > 1 and logits.stride(0) % V:
        raise ValueError("logits row pitch must be a multiple of the vocabulary")
    pitch = logits.stride(0) if B > 1 else V
    _check_extent(logits, (B - 1) * pitch + V, "logits")
    if noise.dtype != torch.float32 or not noise.is_contiguous() or noise.numel() != B * V:
        raise ValueError("noise must be a contiguous float32 (batch, vocab) tensor")
    temperature = temperature.to(device=dev, dtype=torch.float32).contiguous()
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=dev)
    if out.dtype != torch.int32 or out.dim() != 1 or out.numel() != B:
        raise ValueError("out must be an int32 (batch,) tensor")
    h = _lib.lib()
    code = _lib.dtype_code(logits.dtype)
    nbytes = int(h.nsv_sample_workspace_size(B, V, code))
    ws = _lib.workspace(dev, nbytes, "sample")
    rc = h.nsv_sample(logits.data_ptr(), pitch, temperature.data_ptr(), noise.data_ptr(), B, V, code, out.data_ptr(),
                      out.stride(0) if B > 1 else 1, _lib.ptr(ws), nbytes, _lib.stream_ptr(dev))
    _lib.check(rc, "sample")
    return out


def draw_randomness(num_drafts: list[int], V: int, dtype: torch.dtype, device, with_draft_rows: bool,
                    generator: torch.Generator | None = None,
                    active: list[bool] | None = None) -> tuple[torch.Tensor | None, torch.Tensor]:
    """Draw, sequence by sequence, what the reference's verify_stochastic
    draws from ``generator``: rand(K_b) then the exponential noise of its
    multinomial ([V] with draft rows, [K_b+1, V] without).  Sequences with
    active[b] False (greedy ones) draw nothing, as in the reference.
    Returns padded (uniforms [B, K] fp32 or None, noise [B, V] or
    [B, K+1, V])."""
    B, K = len(num_drafts), max(num_drafts) if num_drafts else 0
    u = torch.zeros(B, K, dtype=torch.float32, device=device) if with_draft_rows else None
    if with_draft_rows:
        q = torch.ones(B, V, dtype=dtype, device=device)
    else:
        q = torch.ones(B, K + 1, V, dtype=dtype, device=device)
    for b, k in enumerate(num_drafts):
        if active is not None and not active[b]:
            continue
        if with_draft_rows:
            u[b, :k] = torch.rand(k, device=device, generator=generator)
            q[b] = torch.empty(V, dtype=dtype, device=device).exponential_(1, generator=generator)
        else:
            q[b, :k + 1] = torch.empty(k + 1, V, dtype=dtype, device=device).exponential_(1, generator=generator)
    return u, q


class RejectionSampler:
    """Drop-in for src/myvllm/spec_engine/rejection_sampler.py:24-98.  The
    per-sequence calls launch the batched kernels with one sequence and
    return a host list, as the reference does."""

    def verify_greedy(self, draft_tokens, target_rows) -> list[int]:
        """target_rows: (K+1, vocab) logits on the GPU, or a ready (K+1,)
        token list (rejection_sampler.py:27-28)."""
        if isinstance(target_rows, list):
            accepted = []
            for drafted, target in zip(draft_tokens, target_rows):
                if drafted != target:
                    return accepted + [target]
                accepted.append(drafted)
            return accepted + [target_rows[len(draft_tokens)]]
        K = len(draft_tokens)
        target_rows = target_rows.contiguous()
        drafts, nd = _pad_drafts([list(draft_tokens)], K, target_rows.device)
        tokens, n = accept_greedy(target_rows, drafts, nd, seq_stride=K + 1)
        return tokens[0, :int(n[0])].tolist()

    def verify_stochastic(self, draft_tokens, target_rows: torch.Tensor, draft_rows: torch.Tensor | None,
                          temperature: float, generator: torch.Generator | None = None) -> list[int]:
        """target_rows: (K+1, vocab); draft_rows: (K, vocab) or None."""
        K = len(draft_tokens)
        target_rows = target_rows.contiguous()
        dev = target_rows.device
        u, q = draw_randomness([K], target_rows.shape[-1], target_rows.dtype, dev, draft_rows is not None, generator)
        drafts, nd = _pad_drafts([list(draft_tokens)], K, dev)
        temp = torch.full((1,), float(temperature), dtype=torch.float32, device=dev)
        drow = 1
        if draft_rows is not None:
            # the reference's fast path hands (K, V) views of a (K, batch, V)
            # buffer: rows are contiguous, the row pitch is batch * V
            V = target_rows.shape[-1]
            if draft_rows.dim() != 2 or draft_rows.stride(-1) != 1 or (K > 1 and draft_rows.stride(0) % V):
                draft_rows = draft_rows.contiguous()
            drow = draft_rows.stride(0) // V if K > 1 else 1
        tokens, n = accept_stochastic(target_rows, drafts, nd, temp, q, uniforms=u, draft_logits=draft_rows,
                                      target_seq_stride=K + 1, draft_seq_stride=0, draft_row_stride=drow)
        return tokens[0, :int(n[0])].tolist()

    def verify(self, draft_tokens, target_rows, draft_rows=None, temperature: float = 0.0,
               generator: torch.Generator | None = None) -> list[int]:
        if temperature <= GREEDY_TEMPERATURE:
            return self.verify_greedy(draft_tokens, target_rows)
        return self.verify_stochastic(draft_tokens, target_rows, draft_rows, temperature, generator)
