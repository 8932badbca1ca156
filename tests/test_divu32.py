"""The invariant-divisor quotients of the elementwise view index maps
(pjrt-ocl_amd/csrc/vm_divu32.h), checked on the CPU: the header's own text is
compiled with g++ and every quotient is compared with C's `/` for divisors 1..4096,
every power of two and its neighbours, and random divisors up to 2^31, each
against the dividends around multiples of d, the 32-bit edge and random ones."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(ROOT, "pjrt-ocl_amd", "csrc")

HARNESS = r"""
#define VM_HD inline
#include "vm_divu32.h"
#include <cstdio>
#include <random>
#include <vector>
int main() {
  std::vector<uint32_t> ds;
  for (uint32_t d = 1; d <= 4096; ++d) ds.push_back(d);
  for (int k = 1; k < 32; ++k) {
    const uint64_t p = uint64_t(1) << k;
    for (int64_t e = -2; e <= 2; ++e)
      if (p + e >= 1 && p + e <= 0x7FFFFFFFu) ds.push_back(uint32_t(p + e));
  }
  std::mt19937_64 rng(7);
  for (int j = 0; j < 3000; ++j) ds.push_back(1u + uint32_t(rng() % 0x7FFFFFFFu));
  ds.push_back(0x7FFFFFFFu);
  long bad = 0, checked = 0;
  for (uint32_t d : ds) {
    const vm::DivU32 v = vm::div_u32(d);
    std::vector<uint32_t> xs = {0u, 1u, 2u, d - 1, d, d + 1, 2 * d - 1, 2 * d, 0xFFFFFFFFu, 0xFFFFFFFEu,
                                0x80000000u, 0x7FFFFFFFu};
    const uint32_t top = 0xFFFFFFFFu / d;
    for (int j = 0; j < 64; ++j) {
      const uint32_t k = uint32_t(rng() % (uint64_t(top) + 1));
      xs.push_back(k * d);
      xs.push_back(k * d - 1);
      if (k * uint64_t(d) + d - 1 <= 0xFFFFFFFFull) xs.push_back(k * d + d - 1);
      xs.push_back(uint32_t(rng()));
    }
    for (uint32_t x : xs) {
      ++checked;
      if (v.quo(x) != x / d) {
        if (bad < 8) std::printf("d=%u x=%u got %u want %u\n", d, x, v.quo(x), x / d);
        ++bad;
      }
    }
  }
  std::printf("checked %ld bad %ld\n", checked, bad);
  return bad != 0;
}
"""


def test_invariant_divisor_quotients(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    src, exe = tmp_path / "divu32_check.cpp", tmp_path / "divu32_check"
    src.write_text(HARNESS)
    subprocess.run([gxx, "-O2", "-std=c++17", f"-I{HEADER_DIR}", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout
    assert "bad 0" in out.stdout and "checked" in out.stdout
