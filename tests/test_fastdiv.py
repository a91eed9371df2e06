"""The launch-time integer division (csrc/fd_fastdiv.h) used by every row
decomposition equals exact division, checked on the host by brute force (CPU)."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "fused-decode_amd" / "csrc"

PROGRAM = r"""
#include <cstdio>
#include <cstdint>
#include <random>
#include <vector>
#include "fd_fastdiv.h"
int main() {
  std::mt19937_64 rng(1);
  uint64_t checked = 0;
  auto check = [&](uint32_t d, uint32_t n) {
    fd::FastDiv f(d);
    uint32_t r;
    uint32_t q = f.divmod(n, r);
    if (q != n / d || r != n % d) { std::printf("FAIL d=%u n=%u q=%u\n", d, n, q); return false; }
    ++checked;
    return true;
  };
  std::vector<uint32_t> ds;
  for (uint32_t d = 1; d <= 70000; ++d) ds.push_back(d);
  for (int s = 1; s < 32; ++s) { uint32_t p = 1u << s; ds.push_back(p - 1); ds.push_back(p); ds.push_back(p + 1); }
  ds.push_back(0xffffffffu); ds.push_back(0xfffffffeu); ds.push_back(0x80000001u);
  for (int i = 0; i < 20000; ++i) ds.push_back(uint32_t(rng()) | 1u);
  for (uint32_t d : ds) {
    uint32_t ns[] = {0u, 1u, d - 1, d, d + 1, 2 * d - 1, 2 * d, 0xffffffffu, 0xfffffffeu,
                     0x7fffffffu, 0x80000000u, uint32_t(0xffffffffu / d * d), uint32_t(0xffffffffu / d * d - 1)};
    for (uint32_t n : ns) if (!check(d, n)) return 1;
    for (int j = 0; j < 8; ++j) if (!check(d, uint32_t(rng()))) return 1;
  }
  for (uint32_t n = 0; n < 300000; ++n) if (!check(1 + n % 4099, n * 2654435761u)) return 1;
  std::printf("ok %llu\n", (unsigned long long)checked);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_fastdiv_exact(tmp_path):
    src = tmp_path / "fastdiv.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "fastdiv"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("ok ")
