// gemv.hip -- the weight GEMV that picolm offloads through gpu_try_matmul
// (gpu.c:579-702; tensor.c:200-215): out[i] = dot(row i of W, x) for GGUF
// Q4_K, Q6_K and Q8_0 rows, bit-identical to the reference's fused
// dequantize + dot products as its x86-64 build runs them (AVX2 + FMA,
// quant.c:390-452, 517-582, 627-659).
//
// Those products keep eight running sums (one per 256-bit lane), add them as
// ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)) (hsum_avx2, quant.h:33-46) and chain
// the per-block terms into one sum in block order.  Here every GPU lane owns
// whole 256-bit-lane chains of one row slice, in the reference's order; the
// per-term results go to LDS and one lane per row adds them in order.
//
// Weights live on the device in a packed copy made once at upload
// (plh_gemv_upload): the same bytes, rearranged so that every lane reads its
// quants with one aligned vector load (the reference's 210- and 34-byte
// blocks are not 4-byte aligned).  HBM traffic equals the GGUF size.
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "attn_common.h"
#include "picolm_hip.h"
#include "plh_internal.h"

using namespace plh;

namespace {

constexpr int kThreads = 256;
constexpr int kTypeQ8_0 = 8, kTypeQ4K = 12, kTypeQ6K = 14;
constexpr size_t kPlaneAlign = 256;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Packed layouts (d rows, nb blocks per row):
//  Q4_K: the reference's 144-byte blocks, header unchanged; inside each
//        32-byte sub-block the quant byte of 256-bit lane k = 4h + kk at
//        step t (original byte 8t + k) moves to byte 16h + 4t + kk, so a
//        lane owning lanes 4h..4h+3 reads one 16-byte vector.
//  Q6_K: three planes.  Quants [d][nb][16 groups][12 B]: group j holds
//        elements 16j..16j+15 of the block as two words of low nibbles
//        (word w, byte b: element 8w + b low, 8w + b + 4 high) and one word
//        of high bit pairs (byte b, bits 2s: element b + 4s); then the int8
//        scales [d][nb][16] and the fp16 scales [d][nb].
//  Q8_0: the int8 quants [d][nb][32] and the fp16 scales [d][nb].
struct Layout {
  int block_w = 0;       // weights per block
  int nb = 0;            // blocks per row
  size_t q_bytes = 0;    // quant plane bytes per block
  size_t scales_off = 0, d_off = 0, total = 0;
};

bool make_layout(int qtype, int n, int d, Layout& L) {
  if (n <= 0 || d <= 0) return false;
  switch (qtype) {
    case kTypeQ4K: L.block_w = 256; L.q_bytes = 144; break;
    case kTypeQ6K: L.block_w = 256; L.q_bytes = 192; break;
    case kTypeQ8_0: L.block_w = 32; L.q_bytes = 32; break;
    default: return false;
  }
  if (n % L.block_w) return false;
  L.nb = n / L.block_w;
  const size_t blocks = (size_t)d * L.nb;
  size_t off = align_up(blocks * L.q_bytes, kPlaneAlign);
  if (qtype == kTypeQ6K) {
    L.scales_off = off;
    off = align_up(off + blocks * 16, kPlaneAlign);
  }
  if (qtype != kTypeQ4K) {
    L.d_off = off;
    off = align_up(off + blocks * 2, kPlaneAlign);
  }
  L.total = off;
  return true;
}

// The 6-bit value of element e of a reference Q6_K block (quant.c:199-213).
int q6k_value(const uint8_t* blk, int e) {
  const int c = e / 128, r = e % 128, quarter = r / 32, l = r % 32;
  const uint8_t* ql = blk + 64 * c;
  const uint8_t* qh = blk + 128 + 32 * c;
  const int lo = (quarter & 1) ? ql[l + 32] : ql[l];
  const int nib = (quarter & 2) ? (lo >> 4) : (lo & 0x0F);
  return nib | (((qh[l] >> (2 * quarter)) & 3) << 4);
}

void pack_rows(int qtype, const Layout& L, int d, const uint8_t* src, uint8_t* dst) {
  const size_t blocks = (size_t)d * L.nb;
  if (qtype == kTypeQ4K) {
    for (size_t b = 0; b < blocks; ++b) {
      const uint8_t* s = src + b * 144;
      uint8_t* o = dst + b * 144;
      memcpy(o, s, 16);
      for (int j = 0; j < 4; ++j)
        for (int h = 0; h < 2; ++h)
          for (int t = 0; t < 4; ++t)
            for (int kk = 0; kk < 4; ++kk)
              o[16 + 32 * j + 16 * h + 4 * t + kk] = s[16 + 32 * j + 8 * t + 4 * h + kk];
    }
  } else if (qtype == kTypeQ6K) {
    for (size_t b = 0; b < blocks; ++b) {
      const uint8_t* s = src + b * 210;
      uint8_t* o = dst + b * 192;
      for (int j = 0; j < 16; ++j) {
        int v[16];
        for (int e = 0; e < 16; ++e) v[e] = q6k_value(s, 16 * j + e);
        uint8_t* g = o + 12 * j;
        for (int w = 0; w < 2; ++w)
          for (int bb = 0; bb < 4; ++bb)
            g[4 * w + bb] = (uint8_t)((v[8 * w + bb] & 15) | ((v[8 * w + bb + 4] & 15) << 4));
        for (int bb = 0; bb < 4; ++bb) {
          int hb = 0;
          for (int sh = 0; sh < 4; ++sh) hb |= ((v[bb + 4 * sh] >> 4) & 3) << (2 * sh);
          g[8 + bb] = (uint8_t)hb;
        }
      }
      memcpy(dst + L.scales_off + b * 16, s + 192, 16);
      memcpy(dst + L.d_off + b * 2, s + 208, 2);
    }
  } else {  // Q8_0
    for (size_t b = 0; b < blocks; ++b) {
      const uint8_t* s = src + b * 34;
      memcpy(dst + b * 32, s + 2, 32);
      memcpy(dst + L.d_off + b * 2, s, 2);
    }
  }
}

struct GemvArgs {
  const uint8_t* w;     // packed matrix
  const float* x;       // [n]
  float* out;           // [d]
  int d;
  int nb;               // blocks per row
  int units;            // lane units per row
  int uspan;            // units covered by one pass of the threads (<= 256)
  int row_par;          // rows worked side by side (kThreads / uspan)
  int unit_iters;       // passes over the units
  int rows_per_wg;      // rows of one workgroup
  int terms;            // chained terms per row
  int tpitch;           // LDS pitch of a row's terms
  size_t scales_off, d_off;
};

__device__ __forceinline__ float hsum8(const float (&v)[8]) {
  const float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
  return (a0 + a2) + (a1 + a3);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *(const float4*)p; }

// byte b of a word as a float (exact)
__device__ __forceinline__ float ubyte(uint32_t w, int b) {
  return (float)((w >> (8 * b)) & 0xFFu);
}

// ---- Q4_K: a unit is half h of 64-element sub-block s (256-bit lanes
// 4h..4h+3); the pair (s, 0), (s, 1) sits in adjacent lanes -----------------
struct Q4KUnit {
  float xl[4][4], xh[4][4];  // x of the unit's lanes, steps t = 0..3
  float sx1, sx2;            // hsum of the x running sums (row independent)
};

__device__ __forceinline__ void q4k_load_x(const float* x, int u, Q4KUnit& U) {
  const int s = u >> 1, h = u & 1;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const float4 a = ld4(x + 64 * s + 8 * t + 4 * h);
    const float4 b = ld4(x + 64 * s + 32 + 8 * t + 4 * h);
    U.xl[t][0] = a.x, U.xl[t][1] = a.y, U.xl[t][2] = a.z, U.xl[t][3] = a.w;
    U.xh[t][0] = b.x, U.xh[t][1] = b.y, U.xh[t][2] = b.z, U.xh[t][3] = b.w;
  }
  // sum_x1 / sum_x2 (quant.c:433): lane k adds x[k] + x[8+k], then
  // x[16+k] + x[24+k], onto zero
  float s1[4], s2[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    float a = 0.0f + (U.xl[0][kk] + U.xl[1][kk]);
    s1[kk] = a + (U.xl[2][kk] + U.xl[3][kk]);
    float b = 0.0f + (U.xh[0][kk] + U.xh[1][kk]);
    s2[kk] = b + (U.xh[2][kk] + U.xh[3][kk]);
  }
  float p1[4], p2[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    p1[kk] = s1[kk] + __shfl_xor(s1[kk], 1, 64);
    p2[kk] = s2[kk] + __shfl_xor(s2[kk], 1, 64);
  }
  U.sx1 = (p1[0] + p1[2]) + (p1[1] + p1[3]);
  U.sx2 = (p2[0] + p2[2]) + (p2[1] + p2[3]);
}

// get_scale_min_k4 (quant.c:82-91) on the 12 scale bytes held in three words
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                              int& sc, int& mn) {
  auto byte = [&](int i) -> int {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (int)((w >> (8 * (i & 3))) & 0xFFu);
  };
  if (j < 4) {
    sc = byte(j) & 63;
    mn = byte(j + 4) & 63;
  } else {
    sc = (byte(j + 4) & 0x0F) | ((byte(j - 4) >> 6) << 4);
    mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
  }
}

// The term of sub-block s for one row: both lanes of the pair return it.
__device__ __forceinline__ float q4k_term(const uint8_t* row, int u, const Q4KUnit& U) {
  const int s = u >> 1, h = u & 1;
  const int blk = s >> 2, j = s & 3;
  const uint8_t* b = row + (size_t)blk * 144;
  const uint4 hdr = *(const uint4*)b;
  const uint4 q = *(const uint4*)(b + 16 + 32 * j + 16 * h);
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
  float a1[4], a2[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a1[kk] = a2[kk] = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t lo = qw[t] & 0x0F0F0F0Fu, hi = (qw[t] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      a1[kk] = __builtin_fmaf(ubyte(lo, kk), U.xl[t][kk], a1[kk]);
      a2[kk] = __builtin_fmaf(ubyte(hi, kk), U.xh[t][kk], a2[kk]);
    }
  }
  float p1[4], p2[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    p1[kk] = a1[kk] + __shfl_xor(a1[kk], 1, 64);
    p2[kk] = a2[kk] + __shfl_xor(a2[kk], 1, 64);
  }
  const float sqx1 = (p1[0] + p1[2]) + (p1[1] + p1[3]);
  const float sqx2 = (p2[0] + p2[2]) + (p2[1] + p2[3]);
  const float dd = f16_bits_to_f32((uint16_t)(hdr.x & 0xFFFFu));
  const float dmin = f16_bits_to_f32((uint16_t)(hdr.x >> 16));
  int sc, mn;
  q4k_scale_min(2 * j, hdr.y, hdr.z, hdr.w, sc, mn);
  const float d1 = dd * (float)sc, m1 = dmin * (float)mn;
  q4k_scale_min(2 * j + 1, hdr.y, hdr.z, hdr.w, sc, mn);
  const float d2 = dd * (float)sc, m2 = dmin * (float)mn;
  const float t0 = d1 * sqx1, t1 = m1 * U.sx1, t2 = d2 * sqx2, t3 = m2 * U.sx2;
  return ((t0 - t1) + t2) - t3;
}

// ---- Q6_K: a unit is 16-element group s of a row (block s/16, group s%16)
struct Q6KUnit {
  float x[16];
};

__device__ __forceinline__ void q6k_load_x(const float* x, int u, Q6KUnit& U) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 a = ld4(x + 16 * u + 4 * i);
    U.x[4 * i] = a.x, U.x[4 * i + 1] = a.y, U.x[4 * i + 2] = a.z, U.x[4 * i + 3] = a.w;
  }
}

__device__ __forceinline__ float q6k_term(const GemvArgs& a, size_t rblk, int u,
                                          const Q6KUnit& U) {
  const int blk = u >> 4, j = u & 15;
  const size_t b = rblk + blk;               // block index in the matrix
  const uint8_t* g = a.w + b * 192 + 12 * j;
  const uint32_t L0 = *(const uint32_t*)g, L1 = *(const uint32_t*)(g + 4);
  const uint32_t H = *(const uint32_t*)(g + 8);
  const int sc = (int)(int8_t)a.w[a.scales_off + b * 16 + j];
  const float dd = f16_bits_to_f32(*(const uint16_t*)(a.w + a.d_off + b * 2));
  // bytes of v for elements 0-3, 4-7, 8-11, 12-15
  const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x03030303u;
  const uint32_t v0 = (L0 & m4) | ((H & m2) << 4);
  const uint32_t v1 = ((L0 >> 4) & m4) | (((H >> 2) & m2) << 4);
  const uint32_t v2 = (L1 & m4) | (((H >> 4) & m2) << 4);
  const uint32_t v3 = ((L1 >> 4) & m4) | (((H >> 6) & m2) << 4);
  float p[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float fl0 = ubyte(v0, k) - 32.0f, fl1 = ubyte(v1, k) - 32.0f;
    const float fh0 = ubyte(v2, k) - 32.0f, fh1 = ubyte(v3, k) - 32.0f;
    p[k] = __builtin_fmaf(fl0, U.x[k], fh0 * U.x[8 + k]);
    p[4 + k] = __builtin_fmaf(fl1, U.x[4 + k], fh1 * U.x[12 + k]);
  }
  const float ds = dd * (float)sc;
  return ds * hsum8(p);
}

// ---- Q8_0: a unit is one 32-element block ---------------------------------
struct Q80Unit {
  float x[32];
};

__device__ __forceinline__ void q80_load_x(const float* x, int u, Q80Unit& U) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 a = ld4(x + 32 * u + 4 * i);
    U.x[4 * i] = a.x, U.x[4 * i + 1] = a.y, U.x[4 * i + 2] = a.z, U.x[4 * i + 3] = a.w;
  }
}

__device__ __forceinline__ float sbyte(uint32_t w, int b) {
  return (float)(int)(int8_t)((w >> (8 * b)) & 0xFFu);
}

__device__ __forceinline__ float q80_term(const GemvArgs& a, size_t rblk, int u,
                                          const Q80Unit& U) {
  const size_t b = rblk + u;
  const uint4 q0 = *(const uint4*)(a.w + b * 32);
  const uint4 q1 = *(const uint4*)(a.w + b * 32 + 16);
  const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const float dd = f16_bits_to_f32(*(const uint16_t*)(a.w + a.d_off + b * 2));
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    // element 8t + k sits in word 2t + k/4, byte k%4
    const float p0 = sbyte(qw[0 + k / 4], k & 3) * U.x[k];
    const float p1 = sbyte(qw[2 + k / 4], k & 3) * U.x[8 + k];
    const float p2 = sbyte(qw[4 + k / 4], k & 3) * U.x[16 + k];
    const float p3 = sbyte(qw[6 + k / 4], k & 3) * U.x[24 + k];
    acc[k] = (p0 + p1) + (p2 + p3);
  }
  return dd * hsum8(acc);
}

// One workgroup: rows [r0, r0 + rows_per_wg).  Phase 1: thread tid owns unit
// tid % uspan (+ uspan per pass) of rows tid / uspan + row_par * i, keeps the
// unit's x in registers and writes the unit's term per row to LDS.  Phase 2:
// one thread per row adds the row's terms in order.
template <int QT>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
  extern __shared__ float terms[];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.x * a.rows_per_wg;
  const int rows = min(a.rows_per_wg, a.d - r0);
  const int rlane = tid / a.uspan;
  if (rlane < a.row_par) {
    for (int it = 0; it < a.unit_iters; ++it) {
      const int u = tid % a.uspan + it * a.uspan;
      if (u >= a.units) break;  // pairs of Q4_K units leave together (units even)
      if (QT == kTypeQ4K) {
        Q4KUnit U;
        q4k_load_x(a.x, u, U);
        const size_t row_bytes = (size_t)a.nb * 144;
        for (int rr = rlane; rr < rows; rr += a.row_par) {
          const float t = q4k_term(a.w + (size_t)(r0 + rr) * row_bytes, u, U);
          if ((u & 1) == 0) terms[rr * a.tpitch + (u >> 1)] = t;
        }
      } else if (QT == kTypeQ6K) {
        Q6KUnit U;
        q6k_load_x(a.x, u, U);
        for (int rr = rlane; rr < rows; rr += a.row_par)
          terms[rr * a.tpitch + u] = q6k_term(a, (size_t)(r0 + rr) * a.nb, u, U);
      } else {
        Q80Unit U;
        q80_load_x(a.x, u, U);
        for (int rr = rlane; rr < rows; rr += a.row_par)
          terms[rr * a.tpitch + u] = q80_term(a, (size_t)(r0 + rr) * a.nb, u, U);
      }
    }
  }
  __syncthreads();
  if (tid < rows) {
    const float* t = terms + tid * a.tpitch;
    float sumf = 0.0f;
    for (int s = 0; s < a.terms; ++s) sumf = sumf + t[s];
    a.out[r0 + tid] = sumf;
  }
}

}  // namespace

extern "C" {

size_t plh_gemv_packed_bytes(int qtype, int n, int d) {
  Layout L;
  return make_layout(qtype, n, d, L) ? L.total : 0;
}

int plh_gemv_pack_host(int qtype, int n, int d, const void* host_rows, void* host_packed) {
  Layout L;
  if (!make_layout(qtype, n, d, L)) {
    set_error("plh_gemv_pack_host: no GEMV for type %d with n=%d d=%d", qtype, n, d);
    return -1;
  }
  if (!host_rows || !host_packed) {
    set_error("plh_gemv_pack_host: null pointer");
    return -1;
  }
  memset(host_packed, 0, L.total);
  pack_rows(qtype, L, d, (const uint8_t*)host_rows, (uint8_t*)host_packed);
  return 0;
}

int plh_gemv_upload(int qtype, int n, int d, const void* host_rows, void* dev) {
  Layout L;
  if (!make_layout(qtype, n, d, L)) {
    set_error("plh_gemv_upload: no GEMV for type %d with n=%d d=%d", qtype, n, d);
    return -1;
  }
  if (!host_rows || !dev) {
    set_error("plh_gemv_upload: null pointer");
    return -1;
  }
  std::vector<uint8_t> packed(L.total, 0);
  pack_rows(qtype, L, d, (const uint8_t*)host_rows, packed.data());
  Context& c = ctx();
  if (check_hip(hipMemcpyAsync(dev, packed.data(), L.total, hipMemcpyHostToDevice, c.stream),
                "hipMemcpyAsync(gemv weights)"))
    return -1;
  return check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
}

int plh_gemv(int qtype, int n, int d, const void* dev, const float* x, float* out) {
  Layout L;
  if (!make_layout(qtype, n, d, L)) {
    set_error("plh_gemv: no GEMV for type %d with n=%d d=%d", qtype, n, d);
    return -1;
  }
  if (!dev || !x || !out) {
    set_error("plh_gemv: null pointer");
    return -1;
  }
  Context& c = ctx();
  if (!c.stream) {
    set_error("plh_gemv: plh_init has not been called");
    return -1;
  }
  GemvArgs a{};
  a.w = (const uint8_t*)dev;
  a.x = x;
  a.out = out;
  a.d = d;
  a.nb = L.nb;
  a.units = qtype == kTypeQ4K ? n / 32 : (qtype == kTypeQ6K ? n / 16 : n / 32);
  a.terms = qtype == kTypeQ4K ? n / 64 : a.units;
  a.uspan = a.units < kThreads ? a.units : kThreads;
  a.row_par = kThreads / a.uspan;
  a.unit_iters = (a.units + a.uspan - 1) / a.uspan;
  a.tpitch = a.terms + 1;
  a.scales_off = L.scales_off;
  a.d_off = L.d_off;
  // rows per workgroup: a multiple of row_par, at most 64 (the chain phase
  // is one wave) and within 64 KiB of terms, aiming at >= 2 workgroups per CU
  const int cus = c.num_cus > 0 ? c.num_cus : 256;
  int per_thread = 1;
  while (per_thread < 8 && (long)a.row_par * per_thread * 2 * 2 * cus <= d) per_thread *= 2;
  int rows = a.row_par * per_thread;
  const int lds_rows = (int)((64 * 1024) / (sizeof(float) * (size_t)a.tpitch));
  if (rows > 64) rows = 64;
  if (rows > lds_rows) rows = lds_rows;
  if (rows < 1) {
    set_error("plh_gemv: row of %d weights too long for the term buffer", n);
    return -1;
  }
  a.rows_per_wg = rows;
  const size_t lds = sizeof(float) * (size_t)rows * a.tpitch;
  const int grid = (d + rows - 1) / rows;
  switch (qtype) {
    case kTypeQ4K:
      hipLaunchKernelGGL(gemv_kernel<kTypeQ4K>, dim3(grid), dim3(kThreads), lds, c.stream, a);
      break;
    case kTypeQ6K:
      hipLaunchKernelGGL(gemv_kernel<kTypeQ6K>, dim3(grid), dim3(kThreads), lds, c.stream, a);
      break;
    default:
      hipLaunchKernelGGL(gemv_kernel<kTypeQ8_0>, dim3(grid), dim3(kThreads), lds, c.stream, a);
      break;
  }
  return check_hip(hipGetLastError(), "gemv_kernel launch");
}

}  // extern "C"
