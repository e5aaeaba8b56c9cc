"""The decode kernels' multiply-and-shift division (picolm_amd/csrc/fastdiv.h)
on the CPU: the header's constexpr functions are the ones the kernels call,
compiled here by g++ and checked against the machine's integer division.

Divisors: every d below 2^16, d = 2^k - 1, 2^k, 2^k + 1 up to 2^31, and
random ones.  Numerators for each: 0, 1, d - 1, d, d + 1, the multiples
k*d - 1, k*d, k*d + 1 near 2^31 - 1 (where the rounding error of m is
largest), 2^31 - 1, and random values below 2^31."""
import os
import subprocess

from conftest import ROOT

SRC = r"""
#include <stdio.h>
#include <stdlib.h>
#include "fastdiv.h"
using namespace plh;

static unsigned long long state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd31() {
  state ^= state << 13; state ^= state >> 7; state ^= state << 17;
  return (uint32_t)(state >> 33);
}
static long long checked = 0, bad = 0;
static void one(uint32_t n, uint32_t d, FastDiv f) {
  if (n > 0x7fffffffu) return;
  ++checked;
  if (fdiv(n, f) != n / d) {
    if (bad++ < 10) printf("n %u d %u: %u, want %u\n", n, d, fdiv(n, f), n / d);
  }
}
static void divisor(uint32_t d) {
  const FastDiv f = make_fastdiv(d);
  if ((unsigned long long)f.m >= (1ull << 32) || f.sh < 31 || f.sh > 62) {
    ++bad;
    printf("d %u: m %u sh %u out of range\n", d, f.m, f.sh);
  }
  const uint32_t top = 0x7fffffffu;
  const uint32_t edges[] = {0, 1, d - 1, d, d + 1, top};
  for (uint32_t n : edges) one(n, d, f);
  const uint32_t k = top / d;
  for (uint32_t j = 0; j < 3 && j <= k; ++j) {
    const uint32_t base = (k - j) * d;
    one(base - 1, d, f);
    one(base, d, f);
    one(base + 1, d, f);
  }
  for (int i = 0; i < 64; ++i) one(rnd31(), d, f);
  for (int i = 0; i < 16; ++i) one(rnd31() % (d < 65536 ? 65536 * d : top), d, f);
}
int main() {
  static_assert(fdiv(1000, make_fastdiv(7)) == 142, "constexpr evaluation");
  for (uint32_t d = 1; d < 65536; ++d) divisor(d);
  for (int k = 1; k <= 31; ++k) {
    const uint32_t p = 1u << k;
    divisor(p - 1);
    divisor(p);
    if (k < 31) divisor(p + 1);
  }
  for (int i = 0; i < 20000; ++i) divisor(rnd31() | 1u), divisor(rnd31() + 1);
  printf("checked %lld bad %lld\n", checked, bad);
  return bad != 0;
}
"""


def test_fastdiv_matches_integer_division(tmp_path):
    src, exe = tmp_path / "fd.cpp", tmp_path / "fd"
    src.write_text(SRC)
    inc = os.path.join(ROOT, "picolm_amd", "csrc")
    r = subprocess.run(["g++", "-std=c++14", "-O2", "-Wall", "-Werror", "-I" + inc, str(src),
                        "-o", str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    assert "bad 0" in r.stdout
