"""The kernels' division by an invariant divisor (ako_amd/csrc/fastdiv.h):
the host-built constants, applied with the same 32-bit arithmetic as the
device code, against the exact quotient, over every divisor up to 4096, the
powers of two and their neighbours and random 31- and 32-bit divisors, each
with edge and random dividends. Compiled with g++ from the header itself."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "ako_amd" / "csrc"

DRIVER = r"""
#include <cstdio>
#include <random>
#include <utility>
#include <vector>
#include "fastdiv.h"

int main() {
  std::mt19937_64 rng(1234);
  std::vector<uint32_t> divisors;
  for (uint32_t d = 1; d <= 4096; ++d) divisors.push_back(d);
  for (int k = 0; k < 32; ++k) {
    const uint64_t p = uint64_t(1) << k;
    for (int64_t off = -1; off <= 1; ++off) {
      const int64_t d = int64_t(p) + off;
      if (d >= 1 && d <= 0xffffffffLL) divisors.push_back(uint32_t(d));
    }
  }
  for (int i = 0; i < 4000; ++i) divisors.push_back(uint32_t(rng() % 0x7fffffffULL) + 1);
  for (int i = 0; i < 1000; ++i) divisors.push_back(uint32_t(rng() % 0xffffffffULL) + 1);
  long checks = 0, bad = 0;
  for (uint32_t d : divisors) {
    const ako::FastDiv f = ako::make_fastdiv(d);
    uint32_t edge[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 2 * d, 0x7fffffffu, 0x80000000u, 0xfffffffeu,
                       0xffffffffu, 1u << 24, (1u << 24) - 1};
    for (uint32_t n : edge) { ++checks; if (ako::fast_div_host(n, f) != n / d) ++bad; }
    for (int i = 0; i < 200; ++i) {
      const uint32_t n = uint32_t(rng());
      ++checks;
      if (ako::fast_div_host(n, f) != n / d) ++bad;
    }
  }
  // The check has teeth: a constant one too small, or the two shifts
  // swapped, gives wrong quotients.
  long planted = 0;
  for (uint32_t d : {7u, 641u, 1000003u}) {
    ako::FastDiv low = ako::make_fastdiv(d), swapped = low;
    low.m -= 1;
    std::swap(swapped.s1, swapped.s2);
    for (int i = 0; i < 100000; ++i) {
      const uint32_t n = uint32_t(rng());
      planted += ako::fast_div_host(n, low) != n / d;
      planted += ako::fast_div_host(n, swapped) != n / d;
    }
  }
  std::printf("checks=%ld bad=%ld planted=%ld\n", checks, bad, planted);
  return bad == 0 && planted > 0 ? 0 : 1;
}
"""


def test_fast_division_is_exact(tmp_path) -> None:
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not available")
    src = tmp_path / "fastdiv_check.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "fastdiv_check"
    subprocess.run([gxx, "-O2", "-std=c++17", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "bad=0" in out.stdout and int(out.stdout.split("checks=")[1].split()[0]) > 1_000_000
