"""The speculative-decoding drafter / verifier API of the reference's
``myvllm.spec_engine`` package (src/myvllm/spec_engine/__init__.py:1-5),
backed by the gfx950 kernels of libnaivspec.so."""

from naivllm_amd.spec_engine.drafters import NgramDrafter
from naivllm_amd.spec_engine.rejection_sampler import RejectionSampler

__all__ = ["NgramDrafter", "RejectionSampler"]
