"""The fp64 exp of the acceptance kernels (naivllm_amd/csrc/exp_f64.h),
compiled for the CPU from the same header: every table entry is the double
nearest 2^(j/256) (60-digit decimal arithmetic), the reduction constants
split ln2/256 exactly, and over a million seeded arguments in [-745, 0] the
result is within 2 ulps of the 80-bit expl value; 0 and -0 give 1, and
-inf, NaN and arguments past the underflow edge give exactly 0."""

import shutil
import subprocess
from decimal import Decimal, getcontext
from pathlib import Path

import numpy as np
import pytest

HDR = Path(__file__).resolve().parents[1] / "naivllm_amd" / "csrc" / "exp_f64.h"

HARNESS = r"""
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include "exp_f64.h"
static double ulps(double got, long double want) {
  if (want == 0.0L) return got == 0.0 ? 0.0 : 1e30;
  const double w = (double)want;
  const double u = std::nextafter(std::fabs(w), INFINITY) - std::fabs(w);
  return (double)(std::fabs((long double)got - want) / (long double)u);
}
int main() {
  uint64_t s = 0x9e3779b97f4a7c15ull;
  double worst = 0.0, at = 0.0;
  for (int i = 0; i < 1000000; ++i) {
    s ^= s << 13; s ^= s >> 7; s ^= s << 17;
    double t = -745.0 * (double)(s >> 11) / 9007199254740992.0;
    if (i % 4 == 1) t = -30.0 * (double)(s >> 11) / 9007199254740992.0;  // where softmax mass lives
    if (i % 4 == 2) t = -0.02 * (double)(s >> 11) / 9007199254740992.0;  // near the table nodes
    const double got = nsv_exp_nonpos(t, kExp2Frac256);
    const long double want = expl((long double)t);
    if (want < 2.2250738585072014e-308L) continue;  // subnormal results: absolute error only
    const double e = ulps(got, want);
    if (e > worst) { worst = e; at = t; }
  }
  std::printf("%.6f %.17g\n", worst, at);
  const double sp[6] = {0.0, -0.0, -INFINITY, NAN, -745.2, -1e300};
  for (double t : sp) std::printf("%a\n", nsv_exp_nonpos(t, kExp2Frac256));
  return 0;
}
"""


def table_from_header():
    text = HDR.read_text()
    body = text[text.index("kExp2Frac256[256] = {") + len("kExp2Frac256[256] = {"):]
    body = body[:body.index("};")]
    return [float.fromhex(x.strip()) for x in body.split(",") if x.strip()]


def constant(name):
    text = HDR.read_text()
    line = next(l for l in text.splitlines() if f"double {name} =" in l)
    return float.fromhex(line.split("=")[1].split(";")[0].strip())


def test_table_and_split_constants_are_exact():
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    tab = table_from_header()
    assert len(tab) == 256
    for j, v in enumerate(tab):
        assert v == float((Decimal(j) / 256 * ln2).exp()), j
    L = ln2 / 256
    hi, lo = constant("kLhi"), constant("kLlo")
    assert hi == float(L)
    assert lo == float(L - Decimal(hi))
    # L_hi's last bit is 2^-61, which keeps t - k*L_hi exact in one fma
    assert (Decimal(hi) * 2 ** 61) % 1 == 0


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_exp_within_two_ulps(tmp_path):
    src = tmp_path / "h.cpp"
    src.write_text(HARNESS)
    exe = tmp_path / "h"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", f"-I{HDR.parent}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    worst, at = out[0].split()
    assert float(worst) <= 2.0, (worst, at)
    z, nz, ninf, nan, under, far = out[1:7]
    assert float.fromhex(z) == 1.0 and float.fromhex(nz) == 1.0
    assert float.fromhex(ninf) == 0.0 and float.fromhex(under) == 0.0 and float.fromhex(far) == 0.0
    assert float.fromhex(nan) == 0.0
