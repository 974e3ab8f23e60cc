"""Builds libnaivspec.so (the gfx950 HIP kernels behind include/naivspec.h).

Each ``csrc/*.hip`` file is compiled to an object with ``hipcc
--offload-arch=gfx950`` (in parallel), then linked into one shared library
placed next to this file, where ``naivllm_amd._lib`` loads it.  Always
rebuilds: callers use this as the "does it compile" check.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libnaivspec.so")
STAMP_LIB_PATH = os.path.join(PKG_DIR, "libnaivspec_stamp.so")

ARCH = "gfx950"
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # keep the compiler from forming packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; libnaivspec.so cannot be built")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, hipcc: str, build_dir: str, extra: list[str]) -> str:
    obj = os.path.join(build_dir, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *extra, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build_library(verbose: bool = False, stamp: bool = False) -> str:
    """Build libnaivspec.so, or with ``stamp`` its timeline-stamped twin
    libnaivspec_stamp.so (NSV_STAMP=1: the verify-attention kernels record
    per-workgroup clock stamps; see nsv_stamp_configure)."""
    hipcc = _hipcc()
    build_dir = BUILD_DIR + ("_stamp" if stamp else "")
    out = STAMP_LIB_PATH if stamp else LIB_PATH
    extra = ["-DNSV_STAMP=1"] if stamp else []
    os.makedirs(build_dir, exist_ok=True)
    srcs = sources()
    workers = max(1, min(len(srcs), os.cpu_count() or 1, 8))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, hipcc, build_dir, extra), srcs))
    tmp = out + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {os.path.basename(out)} failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(srcs)} sources")
    return out


if __name__ == "__main__":
    import sys

    build_library(verbose=True, stamp="--stamp" in sys.argv[1:])
