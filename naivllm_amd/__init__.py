"""MI355X-native speculative-decoding verification round.

Drop-in for the ``myvllm.spec_engine`` drafter / verifier path of
Hongli-xd/Naivllm, backed by hand-written gfx950 HIP kernels in
libnaivspec.so (C ABI: include/naivspec.h).
"""

__version__ = "0.1.0"
