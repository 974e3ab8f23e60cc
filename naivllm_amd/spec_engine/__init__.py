"""The speculative-decoding drafter / verifier API of the reference's
``myvllm.spec_engine`` package (src/myvllm/spec_engine/__init__.py:1-5),
backed by the gfx950 kernels of libnaivspec.so.  ``SpecLLMEngine`` is
resolved on first access (it imports the device round, which imports the
drafters of this package)."""

from naivllm_amd.spec_engine.drafters import DraftRunner, HybridDrafter, ModelDrafter, NgramDrafter
from naivllm_amd.spec_engine.rejection_sampler import RejectionSampler

__all__ = ["SpecLLMEngine", "NgramDrafter", "ModelDrafter", "RejectionSampler", "HybridDrafter", "DraftRunner"]


def __getattr__(name):
    if name == "SpecLLMEngine":
        from naivllm_amd.spec_engine.spec_llm_engine import SpecLLMEngine
        return SpecLLMEngine
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
