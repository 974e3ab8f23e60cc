"""The C ABI library loads, exports every symbol include/naivspec.h
declares, and rejects bad arguments with the documented codes — all
without touching a GPU (argument checks run before any launch)."""

import os
import re

import pytest

from naivllm_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "naivspec.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(nsv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    h = _lib.lib()
    syms = header_symbols()
    assert syms, "no declarations found"
    for name in syms:
        assert hasattr(h, name), f"{name} declared in naivspec.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_version_and_error_strings():
    h = _lib.lib()
    assert h.nsv_version() >= 100
    assert h.nsv_error_string(0) == b"ok"
    assert h.nsv_error_string(-1) == b"invalid argument"
    assert h.nsv_error_string(-2) == b"unsupported shape"
    assert h.nsv_error_string(-3) == b"workspace missing or too small"


def test_verify_attention_rejects_bad_shapes_before_launch():
    h = _lib.lib()
    base = dict(B=8, T=72, H=16, Hkv=8, D=128, bs=256, mb=6, mq=9, dt=1, split=0)

    def call(**kw):
        a = {**base, **kw}
        return h.nsv_verify_attention(1, 1, 1, 1, 1, 1, 1, 1, 0.1, a["B"], a["T"], a["H"], a["Hkv"], a["D"], a["bs"],
                                      a["mb"], a["mq"], a["dt"], a["split"], None, 0, None)

    assert call(D=96) == -2          # head_dim outside {64, 128}
    assert call(H=12, Hkv=8) == -2   # heads not a multiple of kv heads
    assert call(bs=100) == -2        # page size not a power of two
    assert call(mq=65) == -2         # more than 64 query rows per sequence
    assert call(dt=7) == -1
    assert call(split=100) == -1     # split not a multiple of 128
    assert call(B=-1) == -1
    assert call(split=128) == -3     # 12 key splits need a partials workspace
    assert call(B=0) == 0 and call(T=0) == 0


def test_workspace_size_matches_split_plan():
    h = _lib.lib()
    # config 2 with 128-key splits: 6 pages x 256 keys -> 12 splits of 18 rows: (max, sum) pairs
    # padded to 256 bytes, then 128-float partial rows
    # (a fixed 64 KiB area of per-pair arrival counters first)
    pad = lambda x: (x + 255) // 256 * 256
    rows = 8 * 8 * 12 * 18
    cnt = 65536
    assert h.nsv_verify_attention_workspace_size(8, 16, 8, 128, 256, 6, 9, 1, 128) == cnt + pad(rows * 8) + rows * 512
    # automatic plan for config 2 (6-page tables): the key-split kernel, 64 (sequence, kv-head)
    # pairs x 4 key splits fill the 256 CUs a host without a GPU assumes
    rows = 8 * 8 * 4 * 18
    assert h.nsv_verify_attention_workspace_size(8, 16, 8, 128, 256, 6, 9, 1, 0) == cnt + pad(rows * 8) + rows * 512
    # 4 sequences: 32 pairs take the key-split kernel too, 8 splits each by the CU count (none
    # shorter than 160 keys)
    import ctypes
    kind, splits = ctypes.c_int(), ctypes.c_int()
    assert h.nsv_verify_attention_plan(4, 16, 8, 128, 256, 6, 9, 1, 0, 256, ctypes.addressof(kind),
                                       ctypes.addressof(splits)) == 0
    assert (kind.value, splits.value) == (1, 8)
    rows = 4 * 8 * 8 * 18
    assert h.nsv_verify_attention_workspace_size(4, 16, 8, 128, 256, 6, 9, 1, 0) == cnt + pad(rows * 8) + rows * 512
    # 2 sequences: 16 pairs take it as well; the CU count asks 16 splits, but more than 8 need
    # 512-key splits: 8
    assert h.nsv_verify_attention_plan(2, 16, 8, 128, 256, 6, 9, 1, 0, 256, ctypes.addressof(kind),
                                       ctypes.addressof(splits)) == 0
    assert (kind.value, splits.value) == (1, 8)
    # 1 sequence: 8 pairs keep the d-sliced kernel (4 head-dim slices, key splits merged by a
    # second kernel)
    assert h.nsv_verify_attention_plan(1, 16, 8, 128, 256, 6, 9, 1, 0, 256, ctypes.addressof(kind),
                                       ctypes.addressof(splits)) == 0
    assert kind.value == 0
    # 16-page tables (4096 keys): the key-split kernel, 4 splits per sequence for 64 pairs on
    # the 256 CUs a host without a GPU assumes
    rows = 8 * 8 * 4 * 18
    assert h.nsv_verify_attention_workspace_size(8, 16, 8, 128, 256, 16, 9, 1, 0) == cnt + pad(rows * 8) + rows * 512
    # 16 sequences x 8 kv heads, 128-page tables (config 4's shape at 16 Q heads): 2 splits each
    rows = 16 * 8 * 2 * 18
    assert (h.nsv_verify_attention_workspace_size(16, 16, 8, 128, 256, 128, 9, 1, 0)
            == cnt + pad(rows * 8) + rows * 512)
    # 32 sequences: the pairs fill the chip, one split each, no workspace
    assert h.nsv_verify_attention_workspace_size(32, 16, 8, 128, 256, 6, 9, 1, 0) == 0
    # one split: no workspace
    assert h.nsv_verify_attention_workspace_size(1, 16, 8, 128, 256, 1, 9, 1, 256) == 0


def test_plan_serves_large_groups_in_head_subsets():
    # (H / Hkv) * max_q_len > 64: the plan takes the largest divisor of the group whose
    # rows fit, and sizes the workspace for one subset's rows (the launches share it)
    import ctypes
    h = _lib.lib()
    kind, splits = ctypes.c_int(), ctypes.c_int()
    for H, mq in [(32, 17), (64, 9), (64, 33), (8, 64)]:
        assert h.nsv_verify_attention_plan(2, H, 8, 128, 256, 24, mq, 1, 0, 256, ctypes.addressof(kind),
                                           ctypes.addressof(splits)) == 0, (H, mq)
    # GQA-4 x 17 rows: 2 heads (34 rows) per launch; 24-page tables -> key-split, 16 splits asked
    # for 16 pairs, 12 of at least 512 keys
    rows = 2 * 8 * 12 * 34
    pad = lambda x: (x + 255) // 256 * 256
    assert h.nsv_verify_attention_workspace_size(2, 32, 8, 128, 256, 24, 17, 1, 0) == 65536 + pad(rows * 8) + rows * 512


def test_store_kv_rejects_bad_arguments():
    h = _lib.lib()
    assert h.nsv_store_kv(1, 1, 1, 1, 1, 4, 8, 128, 16, 5, None) == -1
    assert h.nsv_store_kv(None, 1, 1, 1, 1, 4, 8, 128, 16, 1, None) == -1
    assert h.nsv_store_kv(1, 1, 1, 1, 1, 4, 1, 4, 16, 1, None) == -2   # 8-byte rows
    assert h.nsv_store_kv(1, 1, 1, 1, 1, 0, 8, 128, 16, 1, None) == 0


def test_wrappers_raise_value_error_on_rejected_arguments():
    with pytest.raises(ValueError):
        _lib.check(-2, "op")
    with pytest.raises(_lib.NaivspecError):
        _lib.check(1, "op")


def test_accept_and_ngram_reject_bad_arguments_before_launch():
    h = _lib.lib()
    # K above 63 (K + 1 rows must fit one 64-lane wave), bad dtype, stride below K + 1, missing workspace
    assert h.nsv_accept_greedy(1, 65, 1, 1, 2, 64, 100, 1, 1, 1, 1, 1 << 20, None) == -1
    assert h.nsv_accept_workspace_size(2, 64, 100, 1, 1) == 0 and h.nsv_accept_workspace_size(2, 63, 100, 1, 1) > 0
    assert h.nsv_accept_greedy(1, 9, 1, 1, 2, 8, 100, 5, 1, 1, 1, 1 << 20, None) == -1
    assert h.nsv_accept_greedy(1, 8, 1, 1, 2, 8, 100, 1, 1, 1, 1, 1 << 20, None) == -1
    assert h.nsv_accept_greedy(1, 9, 1, 1, 2, 8, 100, 1, 1, 1, None, 0, None) == -3
    assert h.nsv_accept_greedy(1, 9, 1, 1, 0, 8, 100, 1, 1, 1, None, 0, None) == 0   # empty batch
    assert h.nsv_accept_workspace_size(2, 8, 100, 1, 0) > 0
    assert h.nsv_accept_workspace_size(2, 8, 100, 1, 1) > h.nsv_accept_workspace_size(2, 8, 100, 1, 0)
    # stochastic: model mode needs uniforms; a draft_mode array needs draft rows; noise stride too short
    assert h.nsv_accept_stochastic(1, 9, 1, 9, 1, None, 1, 1, 1, None, 1, 0, 2, 8, 100, 1, 1, 1, 1, 1 << 30,
                                   None) == -1
    assert h.nsv_accept_stochastic(1, 9, None, 0, 1, 1, 1, 1, 1, None, 1, 0, 2, 8, 100, 1, 1, 1, 1, 1 << 30,
                                   None) == -1
    assert h.nsv_accept_stochastic(1, 9, 1, 9, 1, 1, 1, 1, 1, 1, 1, 100, 2, 8, 100, 1, 1, 1, 1, 1 << 30,
                                   None) == -1
    # sampler: row stride not a multiple of V, missing workspace, empty batch
    assert h.nsv_sample(1, 150, 1, 1, 2, 100, 1, 1, 1, 1, 1 << 20, None) == -1
    assert h.nsv_sample(1, 100, 1, 1, 2, 100, 1, 1, 1, None, 0, None) == -3
    assert h.nsv_sample(1, 100, 1, 1, 0, 100, 1, 1, 1, None, 0, None) == 0
    assert h.nsv_sample_workspace_size(2, 100, 1) > 0
    # draft-step metadata: K must be >= 1
    assert h.nsv_prepare_draft(1, 8, 1, 1, 2, 16, 1, 2, 0, 1, 1, 1, 1, 1, 1, None) == -1
    assert h.nsv_prepare_draft(1, 8, 1, 1, 2, 16, 1, 0, 4, 1, 1, 1, 1, 1, 1, None) == 0
    # n-gram drafter: n range and continuation length
    assert h.nsv_ngram_draft(1, 1, 10, 2, 0, 4, 8, 1, 1, None) == -1
    assert h.nsv_ngram_draft(1, 1, 10, 2, 3, 2, 8, 1, 1, None) == -1
    assert h.nsv_ngram_draft(1, 1, 10, 2, 2, 65, 8, 1, 1, None) == -1
    assert h.nsv_ngram_draft(1, 1, 10, 2, 2, 4, 0, 1, 1, None) == -1
    assert h.nsv_ngram_draft(1, 1, 10, 0, 2, 4, 8, 1, 1, None) == 0


def test_linear_rejects_bad_arguments_before_launch():
    h = _lib.lib()
    # x, norm_w, ss_in, nss_in, eps, weight, y, resid, ss_out, M, N, K, epilogue, workspace, ws_bytes, stream
    assert h.nsv_linear(1, None, None, 0, 1e-6, 1, 1, None, None, 9, 1000, 1024, 0, None, 0, None) == -2  # N % 16
    assert h.nsv_linear(1, None, None, 0, 1e-6, 1, 1, None, None, 9, 1024, 1020, 0, None, 0, None) == -2  # K % 8
    assert h.nsv_linear(None, None, None, 0, 1e-6, 1, 1, None, None, 9, 1024, 1024, 0, None, 0, None) == -1
    assert h.nsv_linear(1, None, None, 0, 1e-6, 1, 1, None, None, 9, 1024, 1024, 3, None, 0, None) == -1
    assert h.nsv_linear(1, 1, None, 0, 1e-6, 1, 1, None, None, 9, 1024, 1024, 0, None, 0, None) == -1  # norm, no sums
    assert h.nsv_linear(1, None, None, 0, 1e-6, 1, None, None, None, 9, 1024, 1024, 2, None, 0, None) == -1
    assert h.nsv_linear(1, None, None, 0, 1e-6, 1, 1, None, None, 0, 1024, 1024, 0, None, 0, None) == 0  # no rows
    # split reduction (72 rows, 64 column tiles) needs the workspace; 9 rows do not
    assert h.nsv_linear_workspace_size(9, 1024, 2048) == 0
    # residual partial sums: per 8-column tile at few rows over few tiles, else per 16-column tile
    assert h.nsv_linear_ss_rows(9, 1024, 2048, 0) == 256  # 4-column tiles (no device: 256 CUs assumed)
    assert h.nsv_linear_ss_rows(9, 1024, 2048, 1) == 64
    assert h.nsv_linear_ss_rows(18, 1024, 2048, 0) == 256
    assert h.nsv_linear_ss_rows(36, 1024, 2048, 0) == 64
    assert h.nsv_linear_ss_rows(9, 4096, 1024, 0) == 256
    n = h.nsv_linear_workspace_size(72, 1024, 2048)
    assert n >= 64 * 4 * 80 * 16 * 4
    assert h.nsv_linear(1, None, None, 0, 1e-6, 1, 1, None, None, 72, 1024, 2048, 0, None, 0, None) == -3
    assert h.nsv_linear_workspace_size(72, 4096, 1024) == 0  # 256 tiles cover the chip without a split


def linear_plan(M, N, K, norm, epi, cus):
    import ctypes
    cols, ks, half = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = _lib.lib().nsv_linear_plan(M, N, K, int(norm), epi, cus, ctypes.addressof(cols), ctypes.addressof(ks),
                                    ctypes.addressof(half))
    assert rc == 0
    return cols.value, ks.value, half.value


def test_linear_split_only_with_16_column_tiles():
    """A split reduction (ks > 1) is merged only by the 16-column kernel: the
    8- and 32-column kernels deal the reduction to one workgroup.  Sweep the
    dispatch over shapes and CU counts, including partitions with fewer than
    128 CUs, where wide SwiGLU grids and split reductions could both apply."""
    h = _lib.lib()
    seen = set()
    for cus in (20, 38, 64, 80, 100, 127, 128, 200, 256, 304):
        for M in (1, 9, 16, 17, 31, 32, 33, 48, 72, 80, 81, 160):
            for N in (256, 1024, 1536, 2048, 3072, 4096, 6144, 12288, 24576):
                for K in (256, 1024, 2048, 4096):
                    for norm in (False, True):
                        for epi in (0, 1, 2):
                            cols, ks, half = linear_plan(M, N, K, norm, epi, cus)
                            seen.add((cols, ks > 1))
                            assert cols in (4, 8, 16, 32)
                            if cols != 16:
                                assert ks == 1, (cus, M, N, K, norm, epi, cols, ks)
                            if cols == 32:
                                assert epi == 1 and N // 16 >= 128
                            if cols in (4, 8):
                                assert not norm and epi != 1 and M <= 31
                            if cols == 4:
                                assert N // 4 <= cus and half == 0
                            ws = h.nsv_linear_workspace_size(M, N, K)
                            assert (ws > 0) == (ks > 1), (cus, M, N, K, ks, ws)
    assert {(4, False), (8, False), (16, False), (16, True), (32, False)} <= seen


def test_linear_plan_streams_wide_heads():
    """A vocabulary-wide plain projection streams whole tiles per wave
    (half_chunks 2) while its activations fit the LDS; past that, or with a
    prologue or epilogue, the tiled kernels."""
    assert linear_plan(9, 151936, 1024, False, 0, 256) == (16, 1, 2)
    assert linear_plan(72, 151936, 1024, False, 0, 256) == (16, 1, 2)
    assert linear_plan(19, 151936, 4096, False, 0, 256) == (16, 1, 2)
    assert linear_plan(80, 151936, 1024, False, 0, 256)[2] != 2   # 80 x 1032 bf16 > 160 KiB
    assert linear_plan(20, 151936, 4096, False, 0, 256)[2] != 2
    assert linear_plan(9, 151936, 1024, True, 0, 256)[2] != 2    # RMSNorm prologue
    assert linear_plan(9, 151936, 1536, False, 0, 256)[2] != 2   # K outside {1024, 2048, 4096}
    assert linear_plan(9, 4096, 1024, False, 0, 256)[2] != 2     # 256 tiles: too few per CU


def test_linear_plan_rejects_bad_shapes():
    import ctypes
    x = ctypes.c_int()
    h = _lib.lib()
    p = ctypes.addressof(x)
    assert h.nsv_linear_plan(9, 100, 1024, 0, 0, 256, p, p, p) == -1  # N not a multiple of 16
    assert h.nsv_linear_plan(9, 1024, 1020, 0, 0, 256, p, p, p) == -1  # K not a multiple of 8
    assert h.nsv_linear_plan(9, 1024, 1024, 0, 3, 256, p, p, p) == -1  # no epilogue 3


def test_lm_head_rows_and_argument_checks():
    # host-side checks only: nothing is launched (no GPU here: 256 CUs assumed)
    h = _lib.lib()
    assert h.nsv_lm_head_rows(151936, 1024) == 79   # 79 x (1024 + 8) bf16 within 160 KiB of LDS
    assert h.nsv_lm_head_rows(151936, 2048) == 39
    assert h.nsv_lm_head_rows(151936, 4096) == 19
    assert h.nsv_lm_head_rows(151936, 512) == 0     # K not streamed
    assert h.nsv_lm_head_rows(4096, 1024) == 0      # fewer than 32 tiles per CU
    assert h.nsv_lm_head_rows(151930, 1024) == 0    # N not a multiple of 16
    assert h.nsv_lm_head(None, None, None, 0, 151936, 1024, None) == 0  # no rows: nothing to do
    assert h.nsv_lm_head(None, None, None, 9, 151936, 1024, None) == -1
    assert h.nsv_lm_head(1, 1, 1, 80, 151936, 1024, None) == -2         # past the row limit
    assert h.nsv_lm_head_pack(1, 1, 151936, 1000, None) == -2
    assert h.nsv_lm_head_pack(1, 1, 151936, 1024, None) == -1            # in place


def test_no_alloc_entry_rejects_shapes_beyond_its_scratch():
    # a 64-sequence fp32 batch over 128-page tables needs ~19 MB of split
    # partials, beyond the allocation-free entry point's 16 MiB: rejected
    # before anything is launched (no device pointer is touched)
    h = _lib.lib()
    assert h.nsv_verify_attention_noalloc_max_scratch() == 16 << 20
    need = h.nsv_verify_attention_workspace_size(64, 16, 8, 128, 256, 128, 9, 0, 0)
    assert need > 16 << 20
    rc = h.nsv_verify_attention_noalloc(1, 1, 1, 1, 1, 1, 1, 1, 0.1, 64, 576, 16, 8, 128, 256, 128, 9, 0, 0, None)
    assert rc == -4
    assert h.nsv_error_string(-4) == b"shape needs more scratch than the allocation-free entry point holds"
    # shapes the plan refuses keep their own codes
    assert h.nsv_verify_attention_noalloc(1, 1, 1, 1, 1, 1, 1, 1, 0.1, 8, 72, 16, 8, 96, 256, 6, 9, 1, 0, None) == -2
