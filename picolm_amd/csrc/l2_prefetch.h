// l2_prefetch.h -- warming each XCD's L2 with the operands of a later launch.
//
// The eight XCDs of an MI355X each have their own L2, and the dispatcher
// deals a launch's workgroups to them in turn: workgroup c runs on XCD c % 8
// (plh_init checks this).  A weight GEMV's workgroup c reads one contiguous
// byte range of each plane of its matrix, the same for every token, so a
// launch that runs before it with CUs to spare can load those ranges on the
// right XCDs beforehand; read-only lines stay in an XCD's L2 from one launch
// to the next, and the GEMV then streams its weights from L2 instead of HBM.
// One load per 128-byte line is enough to bring the line in.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fastdiv.h"

namespace plh {

constexpr int kPfStreams = 16;           // byte streams of one plan
constexpr int kPfMaxPerXcd = 31;         // prefetch workgroups a launch adds per XCD, at most
constexpr int kPfUnit = 16;              // bytes per lane and load

// The later launch's workgroup wg0 + c reads bytes [c * chunk, min((c + 1) *
// chunk, len)) of the stream, on XCD (c + xoff) % 8 (xoff = wg0 % 8):
// nchunks chunks of uc 16-byte units (fd_uc divides by uc).  chunk and len
// are multiples of 16.
struct PfStream {
  const uint8_t* base;
  uint32_t chunk, len, nchunks, uc, xoff;
  FastDiv fd_uc;
};
struct PfPlan {
  int n;        // streams in use (0: no prefetch)
  int per_xcd;  // prefetch workgroups per XCD (set by the launch)
  PfStream s[kPfStreams];
};

// Prefetch workgroups per XCD for a launch of n_main workgroups of its own:
// the CUs it leaves idle, one workgroup each (a CU shared with the launch's
// own workgroups slows them), at most kPfMaxPerXcd; 0 when fewer than 8
// would be left.
inline int pf_per_xcd(int num_cus, long n_main) {
  const long free_cus = (long)num_cus - n_main;
  const long per = free_cus / 8 < kPfMaxPerXcd ? free_cus / 8 : kPfMaxPerXcd;
  return per >= 8 ? (int)per : 0;
}

// A launch's prefetch: its workgroups n_main .. n_main + 8 * plan.per_xcd - 1
// take plan.  A kernel argument of its own, so that launches without a plan
// keep the smaller argument block.
struct PfLaunch {
  int n_main;
  PfPlan plan;
};

// LDS a prefetch workgroup needs: 1 KB that the loads land in, then the
// plan's stream descriptors.
constexpr int kPfLdsBytes = 1024 + kPfStreams * (int)sizeof(PfStream);
static_assert(sizeof(PfStream) % 4 == 0, "descriptors are copied as words");

inline bool make_pf_stream(const uint8_t* base, size_t chunk, size_t len, int wg0,
                           PfStream& st) {
  if (chunk == 0 || chunk % kPfUnit || len % kPfUnit || len >= (1ull << 31) ||
      (uintptr_t)base % kPfUnit)
    return false;
  const uint32_t uc = (uint32_t)(chunk / kPfUnit);
  st = PfStream{base,         (uint32_t)chunk, (uint32_t)len, (uint32_t)((len + chunk - 1) / chunk),
                uc,           (uint32_t)(wg0 & 7), make_fastdiv(uc)};
  return true;
}

// A prefetch workgroup of rank `rank` (below pf.per_xcd) on XCD x,
// with `waves` waves, called by all of the workgroup's threads (it has a
// barrier).  The stream
// descriptors are first copied to the LDS in one round of loads (fetched one
// by one from the kernel arguments, each would wait a memory round trip):
// the XCD's lanes take the 16-byte units of the chunks c = c0, c0 + 8, ...
// (c0 = (x - xoff) mod 8) of every stream in turn, consecutive lanes consecutive units, each loaded
// straight into the first 1 KB at `lds` (the workgroup's own LDS, at least
// kPfLdsBytes, overwritten at will), so no register waits on a load and all
// of a lane's loads are in flight at once; the one wait is at the end,
// before the workgroup's LDS is released.  Every load is in bounds: off <
// len, and off and len are multiples of 16.
__device__ __forceinline__ void l2_prefetch(const PfPlan& pf, uint32_t x, uint32_t rank, int waves,
                                            void* lds) {
  typedef __attribute__((address_space(3))) void* lds_ptr;
  typedef __attribute__((address_space(1))) void* global_ptr;
  PfStream* desc = reinterpret_cast<PfStream*>(static_cast<unsigned char*>(lds) + 1024);
  const int words = pf.n * (int)(sizeof(PfStream) / 4);
  for (int i = threadIdx.x; i < words; i += waves * 64)
    reinterpret_cast<uint32_t*>(desc)[i] = reinterpret_cast<const uint32_t*>(pf.s)[i];
  __syncthreads();
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t r = rank * (uint32_t)waves + (threadIdx.x >> 6);
  const uint32_t step = (uint32_t)(pf.per_xcd * waves) * 64u;
  for (int s = 0; s < pf.n; ++s) {
    const PfStream st = desc[s];
    const uint32_t c0 = (x - st.xoff) & 7u;
    if (st.nchunks <= c0) continue;
    const uint32_t total = ((st.nchunks - c0 + 7) / 8) * st.uc;  // this XCD's units
    for (uint32_t t = r * 64u + lane; t < total; t += step) {
      const uint32_t j = fdiv(t, st.fd_uc), u = t - j * st.uc;
      const uint32_t off = (8 * j + c0) * st.chunk + u * kPfUnit;
      if (off < st.len)
        __builtin_amdgcn_global_load_lds((global_ptr)(st.base + off), (lds_ptr)lds, 16, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
}

// The prefetch role of a launch whose workgroups n_main .. n_main + 8 *
// pf.per_xcd - 1 prefetch: each XCD gets pf.per_xcd of them, whatever
// n_main is.  True for the workgroups that took it.
__device__ __forceinline__ bool l2_prefetch_role(const PfPlan& pf, int n_main, int waves,
                                                 void* lds) {
  if ((int)blockIdx.x < n_main) return false;
  l2_prefetch(pf, blockIdx.x & 7u, (blockIdx.x - (uint32_t)n_main) >> 3, waves, lds);
  return true;
}

}  // namespace plh
