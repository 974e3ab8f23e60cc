"""Every module of the package imports first in a fresh interpreter (no
import cycle depends on the order a caller happens to use)."""

import os
import pkgutil
import subprocess
import sys

import naivllm_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_every_module_imports_first():
    # Python modules only (the C-ABI libraries next to them are not)
    mods = [m.name for m in pkgutil.walk_packages(naivllm_amd.__path__, "naivllm_amd.")
            if not m.name.rsplit(".", 1)[-1].startswith("libnaivspec")]
    assert "naivllm_amd.engine.verify_round" in mods
    code = "import importlib, sys\nfor m in sys.argv[1:]:\n    importlib.import_module(m)\n"
    for m in mods:
        res = subprocess.run([sys.executable, "-c", code, m], cwd=ROOT, capture_output=True, text=True)
        assert res.returncode == 0, f"import {m} first failed:\n{res.stderr[-2000:]}"
    from naivllm_amd.spec_engine import SpecLLMEngine  # noqa: F401
