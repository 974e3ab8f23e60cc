"""Helpers shared by the GPU tests: move a synth.VerifyBatch onto the GPU
and compare against the oracle under the contract's tolerances."""

import numpy as np
import torch

# attention output tolerances: bf16 2e-2 abs / 1e-2 rel, fp32 1e-5
TOL = {"bf16": dict(atol=2e-2, rtol=1e-2), "f32": dict(atol=1e-5, rtol=1e-5)}
TORCH_DTYPE = {"bf16": torch.bfloat16, "f32": torch.float32}


def to_device(vb, device="cuda"):
    dt = TORCH_DTYPE[vb.dtype]

    def f(x):
        return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(device=device, dtype=dt)

    return dict(
        query=f(vb.q), k_cache=f(vb.k_cache), v_cache=f(vb.v_cache),
        block_tables=torch.from_numpy(vb.block_tables).to(device),
        context_lens=torch.from_numpy(vb.context_lens).to(device),
        cu_seqlens_q=torch.from_numpy(vb.cu_seqlens_q).to(device),
        positions=torch.from_numpy(vb.positions).to(device),
    )


def assert_close(got, want, dtype, what=""):
    got = got.float().cpu().numpy().astype(np.float64)
    tol = TOL[dtype]
    err = np.abs(got - want)
    bound = tol["atol"] + tol["rtol"] * np.abs(want)
    bad = err > bound
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} elements outside atol={tol['atol']} "
                           f"rtol={tol['rtol']}; max abs err {err.max():.3e}")
    return float(err.max())
