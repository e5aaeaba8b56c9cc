// fastdiv.h -- division by a launch constant with a multiply and a shift.
//
// n / d for 0 <= n < 2^31 and 1 <= d <= 2^31 (Granlund and Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994,
// Theorem 4.2 with N = 31): with l = ceil(log2 d) and
// m = floor(2^(31+l) / d) + 1, which is below 2^32, n / d equals
// (n * m) >> (31 + l).  Kernel index arithmetic divides by launch constants;
// the GPU has no integer divide, and a general 32-bit division costs ~25
// instructions on a kernel's critical path.  The host computes (m, 31 + l)
// once per launch.  constexpr functions compile for both the host and the
// device, so the header also builds without the HIP compiler.
#pragma once

#include <stdint.h>

namespace plh {

struct FastDiv {
  uint32_t m;
  uint32_t sh;
};

constexpr FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while (l < 31 && (1u << l) < d) ++l;
  return FastDiv{(uint32_t)((1ull << (31 + l)) / d + 1), 31 + l};
}

constexpr uint32_t fdiv(uint32_t n, FastDiv f) {
  return (uint32_t)(((uint64_t)n * f.m) >> f.sh);
}

}  // namespace plh
