"""The gather's stream-K cut arithmetic divides by the launch's workgroup and unit counts with div_by_rcp
(ling-engine_amd/csrc/lq_div.hpp): a float-reciprocal estimate with a one-step correction in place of an integer
division. The header is compiled here for the host with g++ (IEEE binary32 multiply and conversions, as on the
device) and checked against integer division at every multiple boundary (k*d - 1, k*d, k*d + 1) over the domain
the launch guarantees: divisors below 2^19, quotients below 2^21, n + d below 2^31."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "ling-engine_amd", "csrc")

DRIVER = r"""
#include <cstdio>
#include "lq_div.hpp"
int main() {
  long long bad = 0, tests = 0;
  for (int d = 1; d < (1 << 19); d += (d < 4096 ? 1 : 1 + d / 512)) {
    const float rd = 1.f / static_cast<float>(d);
    const long long lim = (1LL << 31) - d;
    for (long long k = 0; k < (1LL << 21); k += (k < 2048 ? 1 : 1 + (k >> 8))) {
      for (int e = -1; e <= 1; ++e) {
        const long long n = k * d + e;
        if (n < 0 || n >= lim || n / d >= (1LL << 21)) continue;
        ++tests;
        if (lq::div_by_rcp(static_cast<int>(n), d, rd) != static_cast<int>(n / d)) {
          if (bad < 5) std::printf("mismatch n=%lld d=%d\n", n, d);
          ++bad;
        }
      }
    }
  }
  std::printf("tests %lld mismatches %lld\n", tests, bad);
  return bad != 0 || tests < 1000000;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_div_by_rcp_exact_at_every_boundary(tmp_path):
    src = tmp_path / "div_check.cpp"
    exe = tmp_path / "div_check"
    src.write_text(DRIVER)
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I", CSRC, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout
