"""ctypes binding of libnaivspec.so (declarations in include/naivspec.h).

The library is loaded after ``import torch`` so that its HIP runtime
dependency (libamdhip64.so.7) resolves to the copy torch already loaded:
one runtime per process, so torch's streams and device pointers are valid
inside the library.  There is no fallback: if the library is missing every
operator raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be imported before the library is loaded)

LIB_NAME = "libnaivspec.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
# The same kernels built with timeline stamps (NSV_STAMP=1), loaded instead
# when NSV_STAMP_LIB=1 is set before the first call (bench.py --stamps).
STAMP_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnaivspec_stamp.so")

NSV_F32 = 0
NSV_BF16 = 1

_c_int, _c_f32, _c_vp, _c_size = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
_c_i64 = ctypes.c_int64

# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES: dict[str, tuple] = {
    "nsv_version": (_c_int, []),
    "nsv_error_string": (ctypes.c_char_p, [_c_int]),
    "nsv_verify_attention_workspace_size": (
        _c_size, [_c_int] * 9),
    "nsv_verify_attention_plan": (_c_int, [_c_int] * 10 + [_c_vp] * 2),
    "nsv_stamp_configure": (_c_int, [_c_vp, _c_int]),
    "nsv_verify_attention": (
        _c_int,
        [_c_vp] * 8 + [_c_f32] + [_c_int] * 10 + [_c_vp, _c_size, _c_vp]),
    "nsv_verify_attention_noalloc_max_scratch": (_c_size, []),
    "nsv_verify_attention_noalloc": (
        _c_int,
        [_c_vp] * 8 + [_c_f32] + [_c_int] * 10 + [_c_vp]),
    "nsv_verify_attention_load_floor": (_c_int, [_c_vp] * 4 + [_c_int] * 6 + [_c_vp, _c_vp]),
    "nsv_stream_read": (_c_int, [_c_vp, _c_size, _c_int, _c_vp, _c_vp]),
    "nsv_store_kv": (_c_int, [_c_vp] * 5 + [_c_int] * 5 + [_c_vp]),
    "nsv_accept_workspace_size": (_c_size, [_c_int] * 5),
    "nsv_accept_greedy": (
        _c_int, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_int] * 4 + [_c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "nsv_accept_stochastic": (
        _c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i64] + [_c_vp] * 6 + [_c_i64] + [_c_int] * 4
        + [_c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "nsv_sample_workspace_size": (_c_size, [_c_int] * 3),
    "nsv_sample": (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp] + [_c_int] * 3 + [_c_vp, _c_i64, _c_vp, _c_size, _c_vp]),
    "nsv_prepare_draft": (
        _c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_int, _c_int] + [_c_vp] * 7),
    "nsv_ngram_draft": (_c_int, [_c_vp, _c_vp, _c_i64] + [_c_int] * 4 + [_c_vp, _c_vp, _c_vp]),
    "nsv_prepare_verify": (
        _c_int, [_c_vp, _c_i64] + [_c_vp] * 4 + [_c_int, _c_int, _c_vp, _c_int, _c_int] + [_c_vp] * 5),
    "nsv_rms_norm": (_c_int, [_c_vp] * 5 + [_c_int, _c_int, _c_f32, _c_vp]),
    "nsv_qk_norm_rope_store": (
        _c_int, [_c_vp] * 4 + [_c_int] + [_c_vp] * 5 + [_c_int] * 4 + [_c_f32, _c_vp]),
    "nsv_silu_mul": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_vp]),
    "nsv_embed_rms_norm": (
        _c_int, [_c_vp, _c_vp, _c_i64, _c_vp, _c_f32, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_int, _c_int,
                 _c_vp, _c_vp]),
    "nsv_linear_workspace_size": (_c_size, [_c_int] * 3),
    "nsv_linear_ss_rows": (_c_int, [_c_int] * 4),
    "nsv_linear_plan": (_c_int, [_c_int] * 6 + [_c_vp] * 3),
    "nsv_linear": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_f32, _c_vp, _c_vp, _c_vp, _c_vp] + [_c_int] * 4
                   + [_c_vp, _c_size, _c_vp]),
    "nsv_linear_decode": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_f32, _c_vp, _c_vp, _c_vp, _c_vp]
                          + [_c_int] * 4 + [_c_vp]),
    "nsv_linear_decode_ss_rows": (_c_int, [_c_int] * 2),
    "nsv_lm_head_rows": (_c_int, [_c_int] * 2),
    "nsv_lm_head_pack": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_vp]),
    "nsv_lm_head": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_vp]),
    "nsv_commit": (
        _c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64] + [_c_vp] * 5 + [_c_int, _c_vp, _c_vp, _c_int, _c_int, _c_vp]),
}

_lib = None


class NaivspecError(RuntimeError):
    """A kernel launch failed inside libnaivspec.so."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = STAMP_LIB_PATH if os.environ.get("NSV_STAMP_LIB") == "1" else LIB_PATH
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build it with naivllm_amd.build.build_library() "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        handle = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Map a library return code onto the reference's error behaviour:
    rejected arguments raise ValueError (the reference asserts / raises
    ValueError on bad inputs), launch failures raise NaivspecError."""
    if rc == 0:
        return
    msg = lib().nsv_error_string(rc).decode()
    if rc < 0:
        raise ValueError(f"{what}: {msg} (code {rc})")
    raise NaivspecError(f"{what}: HIP error {rc}: {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return NSV_F32
    if dtype == torch.bfloat16:
        return NSV_BF16
    raise ValueError(f"unsupported dtype {dtype}; libnaivspec handles float32 and bfloat16")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_workspaces: dict = {}
_retired: list = []


def workspace(device: torch.device, nbytes: int, name: str) -> torch.Tensor | None:
    """Per-(device, operator) scratch buffer, grown on demand and reused by
    every call of that operator on the device (so calls must be ordered on
    one stream, as torch's current stream orders them).

    Buffers start zero-filled: verify attention keeps per-pair arrival
    counters at the front of its workspace, which every call leaves at zero.
    A buffer replaced by a larger one is kept alive, so a graph captured
    with the old one never points at freed memory."""
    if nbytes <= 0:
        return None
    key = (device.type, device.index if device.index is not None else torch.cuda.current_device(), name)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 2 * (buf.numel() if buf is not None else 0))
        size = (size + 255) // 256 * 256
        if buf is not None:
            _retired.append(buf)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf
