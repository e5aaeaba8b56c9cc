// gemv.hip -- the weight GEMV that picolm offloads through gpu_try_matmul
// (gpu.c:579-702; tensor.c:200-215): out[i] = dot(row i of W, x) for GGUF
// Q4_K, Q6_K and Q8_0 rows, bit-identical to the reference's fused
// dequantize + dot products as its x86-64 build runs them (AVX2 + FMA,
// quant.c:390-452, 517-582, 627-659).
//
// Those products keep eight running sums (one per 256-bit lane), add them as
// ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)) (hsum_avx2, quant.h:33-46) and chain
// the per-block terms into one sum in block order.  Here every GPU lane owns
// all eight 256-bit-lane chains of one row slice (a Q4_K sub-block, one to
// four Q6_K groups, a Q8_0 block), in the reference's order; the per-term
// results go to LDS and one lane per row adds them in order.
//
// The kernel is VALU-bound near the HBM roof (a weight costs a conversion and
// a fused multiply-add at least), so the packed device copy made at upload
// (plh_gemv_upload) is arranged for few instructions: vector loads that are
// contiguous across adjacent lanes, quant bytes converted straight to float
// (v_cvt_f32_ubyte0..3), 32-bit plane offsets.  The bytes are the GGUF
// bytes rearranged: HBM traffic equals the GGUF size.
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "attn_common.h"
#include "attn_decode_dev.h"
#include "picolm_hip.h"
#include "plh_internal.h"

using namespace plh;

namespace plh {
int g_gemv_rows_per_thread = 0;
int g_gemv_exact = 0;
}

namespace {

constexpr int kThreads = 256;
constexpr int kTypeQ8_0 = 8, kTypeQ4K = 12, kTypeQ6K = 14;
constexpr size_t kPlaneAlign = 256;
constexpr size_t kMaxPacked = (size_t)1 << 31;  // 32-bit plane offsets
constexpr int kMaxNormN = kGemvNormMax;          // squares + staged x within 64 KiB of LDS
constexpr int kNormPrefetch = 16;                // x elements per thread loaded up front

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Packed layouts (d rows, nb blocks per row); every plane is row-major over
// the matrix and starts 256-byte aligned:
//  Q4_K: headers [d*nb][16 B] (fp16 d, fp16 dmin, 12 scale bytes), then the
//        quants of each 64-element sub-block in two planes [d*nb*4][16 B]
//        (bytes 0-15 and 16-31 of the reference's 32-byte sub-block).
//  Q6_K: per 16-element group g (row-major over the matrix) two words of low
//        nibbles (L0, L1: word w, byte b holds element 8w + b low, element
//        8w + b + 4 high) and one word of high bit pairs (H: byte b, bits 2s
//        hold element b + 4s), each in its own plane [d*n/16] of words; then
//        the int8 scales [d*n/16] and the fp16 super-block scales [d*nb].
//  Q8_0: quants 0-15 and 16-31 of every block in two planes [d*nb][16 B],
//        then the fp16 scales [d*nb].
struct Layout {
  int block_w = 0;            // weights per block
  int nb = 0;                 // blocks per row
  size_t off[3] = {0, 0, 0};  // plane offsets (Q4_K: header, q0, q1;
                              // Q6_K: L0, L1, H; Q8_0: lo, hi)
  size_t scales_off = 0, d_off = 0, total = 0;
};

bool make_layout(int qtype, int n, int d, Layout& L) {
  if (n <= 0 || d <= 0) return false;
  switch (qtype) {
    case kTypeQ4K: L.block_w = 256; break;
    case kTypeQ6K: L.block_w = 256; break;
    case kTypeQ8_0: L.block_w = 32; break;
    default: return false;
  }
  if (n % L.block_w) return false;
  L.nb = n / L.block_w;
  const size_t blocks = (size_t)d * L.nb;
  if (qtype == kTypeQ4K) {
    L.off[0] = 0;
    L.off[1] = align_up(blocks * 16, kPlaneAlign);
    L.off[2] = L.off[1] + align_up(blocks * 64, kPlaneAlign);
    L.total = L.off[2] + align_up(blocks * 64, kPlaneAlign);
  } else if (qtype == kTypeQ6K) {
    const size_t plane = align_up(blocks * 16 * 4, kPlaneAlign);
    for (int p = 0; p < 3; ++p) L.off[p] = p * plane;
    L.scales_off = 3 * plane;
    L.d_off = align_up(L.scales_off + blocks * 16, kPlaneAlign);
    L.total = align_up(L.d_off + blocks * 2, kPlaneAlign);
  } else {
    const size_t plane = align_up(blocks * 16, kPlaneAlign);
    L.off[0] = 0;
    L.off[1] = plane;
    L.d_off = 2 * plane;
    L.total = align_up(L.d_off + blocks * 2, kPlaneAlign);
  }
  return L.total < kMaxPacked;
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
      memcpy(dst + L.off[0] + b * 16, s, 16);
      for (int j = 0; j < 4; ++j) {
        memcpy(dst + L.off[1] + (b * 4 + j) * 16, s + 16 + 32 * j, 16);
        memcpy(dst + L.off[2] + (b * 4 + j) * 16, s + 32 + 32 * j, 16);
      }
    }
  } else if (qtype == kTypeQ6K) {
    for (size_t b = 0; b < blocks; ++b) {
      const uint8_t* s = src + b * 210;
      for (int j = 0; j < 16; ++j) {
        int v[16];
        for (int e = 0; e < 16; ++e) v[e] = q6k_value(s, 16 * j + e);
        const size_t g = b * 16 + j;  // group index in the matrix
        for (int w = 0; w < 2; ++w)
          for (int bb = 0; bb < 4; ++bb)
            dst[L.off[w] + 4 * g + bb] =
                (uint8_t)((v[8 * w + bb] & 15) | ((v[8 * w + bb + 4] & 15) << 4));
        for (int bb = 0; bb < 4; ++bb) {
          int hb = 0;
          for (int sh = 0; sh < 4; ++sh) hb |= ((v[bb + 4 * sh] >> 4) & 3) << (2 * sh);
          dst[L.off[2] + 4 * g + bb] = (uint8_t)hb;
        }
      }
      memcpy(dst + L.scales_off + b * 16, s + 192, 16);
      memcpy(dst + L.d_off + b * 2, s + 208, 2);
    }
  } else {  // Q8_0
    for (size_t b = 0; b < blocks; ++b) {
      const uint8_t* s = src + b * 34;
      memcpy(dst + L.off[0] + b * 16, s + 2, 16);
      memcpy(dst + L.off[1] + b * 16, s + 18, 16);
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
  int rows_per_wg;      // rows of one workgroup (row_par * rows per thread)
  int terms;            // chained terms per row
  int tpitch;           // LDS pitch of a row's terms
  uint32_t off0, off1, off2, scales_off, d_off;  // plane offsets (bytes)
  // Epilogue, in the reference's order (tensor.c:256-264, 605-657):
  // v = dot; v = v + bias[i] (bias_mode 1) or v + 0.0f (bias_mode 2, a
  // zero-filled bias); v = silu(gate[i]) * v; v = resid[i] + v.
  const float* bias;
  const float* gate;
  const float* resid;
  int bias_mode;
  // Prologue (gemv_kernel<..., true>): x is rmsnorm(x, norm_w) of length n
  // (tensor.c:425-492), formed by every workgroup itself.
  const float* norm_w;
  float norm_eps;
  int n;
  int xs_off;  // floats from the LDS base to the staged rmsnorm(x)
  float* xn_out;  // workgroup 0 also stores rmsnorm(x) here (or null)
  // Gate/up pair (gemv_body<..., true>): virtual row 2r is row r of w (gate),
  // 2r + 1 row r of w2 (up, same type and shape); out[r] = silu(gate) * up.
  const uint8_t* w2;
};

// tensor.c:605-609: x / (1 + expf(-x)).  expf is the device library's, not
// glibc's (which is not correctly rounded), so results can differ from the
// host's in the last place.
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float hsum8(const float (&v)[8]) {
  const float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
  return (a0 + a2) + (a1 + a3);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *(const float4*)p; }

// The x operand as the formats read it, four elements at a time: the vector
// itself, or its rmsnorm (x * scale) * w formed on the fly, rounded as the
// reference's rmsnorm rounds it.
struct PlainX {
  const float* x;
  __device__ __forceinline__ float4 operator()(int i) const { return ld4(x + i); }
};
// rmsnorm(x) staged in LDS by the workgroup, element i at xs_index(i): four
// padding floats after every 64 elements, so that lanes reading the units
// of one row side by side (64 or 32 elements apart) hit different banks.
__host__ __device__ inline int xs_index(int i) { return i + (i >> 6) * 4; }
__host__ __device__ inline int xs_floats(int n) { return xs_index(n) + 4; }
struct LdsX {
  const float* xs;
  __device__ __forceinline__ float4 operator()(int i) const {
    return *(const float4*)(xs + xs_index(i));
  }
};

template <class T>
__device__ __forceinline__ T ld(const uint8_t* w, uint32_t off) {
  return *(const T*)(w + off);
}

// byte B of a word as a float, exact (v_cvt_f32_ubyteB: one instruction)
template <int B>
__device__ __forceinline__ float ubyte(uint32_t w) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
  if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
  if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
  if constexpr (B == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
  return r;
}
__device__ __forceinline__ float ubyte(uint32_t w, int b) {
  switch (b) {
    case 0: return ubyte<0>(w);
    case 1: return ubyte<1>(w);
    case 2: return ubyte<2>(w);
    default: return ubyte<3>(w);
  }
}
__device__ __forceinline__ float sbyte(uint32_t w, int b) {
  return (float)(int)(int8_t)((w >> (8 * b)) & 0xFFu);
}

// ---- Q4_K: a unit is 64-element sub-block s = 4 * block + j ---------------
struct Q4K {
  static constexpr int kTerms = 1;
  struct X {
    float x[64];
    float sx1, sx2;  // hsum of the x running sums (row independent)
  };
  struct Raw {
    uint4 hdr, q0, q1;
  };
  static __device__ __forceinline__ void load_raw(const GemvArgs& a, const uint8_t* w, int row,
                                                  int u, Raw& r) {
    const uint32_t s = (uint32_t)row * a.nb * 4 + u;  // sub-block in the matrix
    r.hdr = ld<uint4>(w, a.off0 + (s >> 2) * 16);
    r.q0 = ld<uint4>(w, a.off1 + s * 16);
    r.q1 = ld<uint4>(w, a.off2 + s * 16);
  }
  template <class XS>
  static __device__ __forceinline__ void load_x(const XS& x, int u, X& U) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float4 v = x(64 * u + 4 * i);
      U.x[4 * i] = v.x, U.x[4 * i + 1] = v.y, U.x[4 * i + 2] = v.z, U.x[4 * i + 3] = v.w;
    }
    // sum_x1 / sum_x2 (quant.c:433): lane k adds x[k] + x[8+k], then
    // x[16+k] + x[24+k], onto zero
    float s1[8], s2[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float a1 = 0.0f + (U.x[k] + U.x[8 + k]);
      s1[k] = a1 + (U.x[16 + k] + U.x[24 + k]);
      const float a2 = 0.0f + (U.x[32 + k] + U.x[40 + k]);
      s2[k] = a2 + (U.x[48 + k] + U.x[56 + k]);
    }
    U.sx1 = hsum8(s1);
    U.sx2 = hsum8(s2);
  }
  // get_scale_min_k4 (quant.c:82-91) on the 12 scale bytes in hdr.y..w
  static __device__ __forceinline__ void scale_min(int j, const uint4& hdr, int& sc, int& mn) {
    auto byte = [&](int i) -> int {
      const uint32_t w = i < 4 ? hdr.y : (i < 8 ? hdr.z : hdr.w);
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
  static __device__ __forceinline__ void terms(int u, const Raw& r, const X& U, float* t) {
    const int j = u & 3;
    // byte 8s + k of the sub-block: word 2s + k/4, byte k%4
    const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    float a1[8], a2[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) a1[k] = a2[k] = 0.0f;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t word = w[2 * st + h];
        const uint32_t lo = word & 0x0F0F0F0Fu, hi = (word >> 4) & 0x0F0F0F0Fu;
        const int k0 = 4 * h;
        const float* xl = U.x + 8 * st + k0;
        const float* xh = U.x + 32 + 8 * st + k0;
        a1[k0 + 0] = __builtin_fmaf(ubyte<0>(lo), xl[0], a1[k0 + 0]);
        a1[k0 + 1] = __builtin_fmaf(ubyte<1>(lo), xl[1], a1[k0 + 1]);
        a1[k0 + 2] = __builtin_fmaf(ubyte<2>(lo), xl[2], a1[k0 + 2]);
        a1[k0 + 3] = __builtin_fmaf(ubyte<3>(lo), xl[3], a1[k0 + 3]);
        a2[k0 + 0] = __builtin_fmaf(ubyte<0>(hi), xh[0], a2[k0 + 0]);
        a2[k0 + 1] = __builtin_fmaf(ubyte<1>(hi), xh[1], a2[k0 + 1]);
        a2[k0 + 2] = __builtin_fmaf(ubyte<2>(hi), xh[2], a2[k0 + 2]);
        a2[k0 + 3] = __builtin_fmaf(ubyte<3>(hi), xh[3], a2[k0 + 3]);
      }
    const float sqx1 = hsum8(a1), sqx2 = hsum8(a2);
    const float dd = f16_bits_to_f32((uint16_t)(r.hdr.x & 0xFFFFu));
    const float dmin = f16_bits_to_f32((uint16_t)(r.hdr.x >> 16));
    int sc, mn;
    scale_min(2 * j, r.hdr, sc, mn);
    const float d1 = dd * (float)sc, m1 = dmin * (float)mn;
    scale_min(2 * j + 1, r.hdr, sc, mn);
    const float d2 = dd * (float)sc, m2 = dmin * (float)mn;
    const float t0 = d1 * sqx1, t1 = m1 * U.sx1, t2 = d2 * sqx2, t3 = m2 * U.sx2;
    t[0] = ((t0 - t1) + t2) - t3;
  }
  static __device__ __forceinline__ int term_index(int u) { return u; }
};

// ---- Q6_K: a unit is G consecutive 16-element groups of one block --------
template <int G>
struct Q6K {
  static constexpr int kTerms = G;
  struct X {
    float x[16 * G];
  };
  struct Raw {
    uint32_t q[3][G];  // L0, L1, H words of the G groups
    uint32_t sc;       // the G int8 scales (low bytes)
    uint32_t d;        // fp16 super-block scale (low half)
  };
  static __device__ __forceinline__ void load_raw(const GemvArgs& a, const uint8_t* w, int row,
                                                  int u, Raw& r) {
    const uint32_t g = (uint32_t)row * a.nb * 16 + (uint32_t)u * G;  // first group
    const uint32_t offs[3] = {a.off0, a.off1, a.off2};
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      if constexpr (G == 4) {
        const uint4 v = ld<uint4>(w, offs[p] + 4 * g);
        r.q[p][0] = v.x, r.q[p][1] = v.y, r.q[p][2] = v.z, r.q[p][3] = v.w;
      } else if constexpr (G == 2) {
        const uint2 v = ld<uint2>(w, offs[p] + 4 * g);
        r.q[p][0] = v.x, r.q[p][1] = v.y;
      } else {
        r.q[p][0] = ld<uint32_t>(w, offs[p] + 4 * g);
      }
    }
    if constexpr (G == 4)
      r.sc = ld<uint32_t>(w, a.scales_off + g);
    else if constexpr (G == 2)
      r.sc = ld<uint16_t>(w, a.scales_off + g);
    else
      r.sc = ld<uint8_t>(w, a.scales_off + g);
    r.d = ld<uint16_t>(w, a.d_off + (g >> 4) * 2);
  }
  template <class XS>
  static __device__ __forceinline__ void load_x(const XS& x, int u, X& U) {
#pragma unroll
    for (int i = 0; i < 4 * G; ++i) {
      const float4 v = x(16 * G * u + 4 * i);
      U.x[4 * i] = v.x, U.x[4 * i + 1] = v.y, U.x[4 * i + 2] = v.z, U.x[4 * i + 3] = v.w;
    }
  }
  // sums[j] of each group (quant.c:559-578), times d * scale (quant.c:581)
  static __device__ __forceinline__ void terms(int, const Raw& r, const X& U, float* t) {
    const float dd = f16_bits_to_f32((uint16_t)(r.d & 0xFFFFu));
    const uint32_t m4 = 0x0F0F0F0Fu, m30 = 0x30303030u;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint32_t L0 = r.q[0][g], L1 = r.q[1][g], H = r.q[2][g];
      // bytes of the 6-bit values of elements 0-3, 4-7, 8-11, 12-15
      const uint32_t v0 = (L0 & m4) | ((H << 4) & m30);
      const uint32_t v1 = ((L0 >> 4) & m4) | ((H << 2) & m30);
      const uint32_t v2 = (L1 & m4) | (H & m30);
      const uint32_t v3 = ((L1 >> 4) & m4) | ((H >> 2) & m30);
      const float* xg = U.x + 16 * g;
      float p[8];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float fl0 = ubyte(v0, k) - 32.0f, fl1 = ubyte(v1, k) - 32.0f;
        const float fh0 = ubyte(v2, k) - 32.0f, fh1 = ubyte(v3, k) - 32.0f;
        p[k] = __builtin_fmaf(fl0, xg[k], fh0 * xg[8 + k]);
        p[4 + k] = __builtin_fmaf(fl1, xg[4 + k], fh1 * xg[12 + k]);
      }
      const float ds = dd * sbyte(r.sc, g);
      t[g] = ds * hsum8(p);
    }
  }
  static __device__ __forceinline__ int term_index(int u) { return u * G; }
};

// ---- Q8_0: a unit is one 32-element block ---------------------------------
struct Q80 {
  static constexpr int kTerms = 1;
  struct X {
    float x[32];
  };
  struct Raw {
    uint4 q0, q1;
    uint32_t d;
  };
  static __device__ __forceinline__ void load_raw(const GemvArgs& a, const uint8_t* w, int row,
                                                  int u, Raw& r) {
    const uint32_t b = (uint32_t)row * a.nb + u;
    r.q0 = ld<uint4>(w, a.off0 + b * 16);
    r.q1 = ld<uint4>(w, a.off1 + b * 16);
    r.d = ld<uint16_t>(w, a.d_off + b * 2);
  }
  template <class XS>
  static __device__ __forceinline__ void load_x(const XS& x, int u, X& U) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 v = x(32 * u + 4 * i);
      U.x[4 * i] = v.x, U.x[4 * i + 1] = v.y, U.x[4 * i + 2] = v.z, U.x[4 * i + 3] = v.w;
    }
  }
  static __device__ __forceinline__ void terms(int, const Raw& r, const X& U, float* t) {
    const uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // element 8s + k sits in word 2s + k/4, byte k%4
      const float p0 = sbyte(qw[0 + k / 4], k & 3) * U.x[k];
      const float p1 = sbyte(qw[2 + k / 4], k & 3) * U.x[8 + k];
      const float p2 = sbyte(qw[4 + k / 4], k & 3) * U.x[16 + k];
      const float p3 = sbyte(qw[6 + k / 4], k & 3) * U.x[24 + k];
      acc[k] = (p0 + p1) + (p2 + p3);
    }
    t[0] = f16_bits_to_f32((uint16_t)(r.d & 0xFFFFu)) * hsum8(acc);
  }
  static __device__ __forceinline__ int term_index(int u) { return u; }
};

// The terms of unit u of the RB rows whose weights are in raw, into LDS.
template <class F, int RB, class XS>
__device__ __forceinline__ void unit_terms(const GemvArgs& a, const XS& xs, float* terms,
                                           int rows, int rlane, int u,
                                           const typename F::Raw (&raw)[RB]) {
  typename F::X U;
  F::load_x(xs, u, U);
#pragma unroll
  for (int k = 0; k < RB; ++k) {
    float t[F::kTerms];
    F::terms(u, raw[k], U, t);
    const int rr = rlane + a.row_par * k;
    if (rr < rows) {
#pragma unroll
      for (int g = 0; g < F::kTerms; ++g) terms[rr * a.tpitch + F::term_index(u) + g] = t[g];
    }
  }
}

// The raw unit u of the RB rows of this thread (rows past the end re-read
// the last row).  PAIR: virtual row v is row v/2 of w (v even) or w2 (odd).
template <class F, int RB, bool PAIR>
__device__ __forceinline__ void load_rows(const GemvArgs& a, int r0, int rows, int rlane, int u,
                                          typename F::Raw (&raw)[RB]) {
#pragma unroll
  for (int k = 0; k < RB; ++k) {
    const int v = r0 + min(rlane + a.row_par * k, rows - 1);
    if constexpr (PAIR)
      F::load_raw(a, (v & 1) ? a.w2 : a.w, v >> 1, u, raw[k]);
    else
      F::load_raw(a, a.w, v, u, raw[k]);
  }
}

// Rows K0 .. K1 - 1 of load_rows.
template <class F, int RB, bool PAIR, int K0, int K1>
__device__ __forceinline__ void load_rows_k(const GemvArgs& a, int r0, int rows, int rlane, int u,
                                            typename F::Raw (&raw)[RB]) {
#pragma unroll
  for (int k = K0; k < K1; ++k) {
    const int v = r0 + min(rlane + a.row_par * k, rows - 1);
    if constexpr (PAIR)
      F::load_raw(a, (v & 1) ? a.w2 : a.w, v >> 1, u, raw[k]);
    else
      F::load_raw(a, a.w, v, u, raw[k]);
  }
}

// Units it0, it0 + 1, ... of this thread (loads of each pass, then terms).
template <class F, int RB, bool PAIR, class XS>
__device__ __forceinline__ void unit_passes(const GemvArgs& a, const XS& xs, float* terms,
                                            int r0, int rows, int rlane, int it0) {
  for (int it = it0; it < a.unit_iters; ++it) {
    const int u = threadIdx.x % a.uspan + it * a.uspan;
    if (u >= a.units) break;
    typename F::Raw raw[RB];
    load_rows<F, RB, PAIR>(a, r0, rows, rlane, u, raw);
    unit_terms<F, RB>(a, xs, terms, rows, rlane, u, raw);
  }
}

// One workgroup: rows [r0, r0 + rows_per_wg).  Phase 1: thread tid owns unit
// tid % uspan (+ uspan per pass) of the RB rows tid / uspan + row_par * k;
// it issues the loads of all RB rows, then loads the unit's x (kept in
// registers for the RB rows) and writes the unit's terms to LDS.  Phase 2:
// one thread per row adds the row's terms in order.  NORM: x is first
// rmsnorm-ed by the workgroup (rms_scale_block, its squares in the LDS that
// the terms take afterwards); the first pass's weight loads are issued
// before, so their latency covers the sum of squares.
template <class F, int RB, bool NORM, bool PAIR>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, int wg, float* terms) {
  const int tid = threadIdx.x;
  const int r0 = wg * a.rows_per_wg;
  const int rows = min(a.rows_per_wg, (PAIR ? 2 * a.d : a.d) - r0);
  const int rlane = tid / a.uspan;
  const bool active = rlane < a.row_par;
  if constexpr (NORM) {
    __shared__ float red[8];
    const int u = tid % a.uspan;
    const bool first = active && u < a.units;
    // x's and the norm weights' loads go first, so that the squares need not
    // wait for the weight loads issued next (loads complete in order);
    // vectors longer than kThreads * kNormPrefetch elements load them after
    float xv[kNormPrefetch], wv[kNormPrefetch];
    const bool pre = a.n <= kThreads * kNormPrefetch;
    if (pre) {
#pragma unroll
      for (int k = 0; k < kNormPrefetch; ++k) {
        const int idx = tid + kThreads * k;
        xv[k] = idx < a.n ? a.x[idx] : 0.0f;
        wv[k] = idx < a.n ? a.norm_w[idx] : 0.0f;
      }
    }
    typename F::Raw raw[RB];
    if (first) load_rows<F, RB, PAIR>(a, r0, rows, rlane, u, raw);
    // lanes 0..7 finish reading the squares before the helper's second
    // barrier, so the terms may overwrite them once it returns
    float scale;
    if (pre) {
      const int lim = 8 * (a.n / 8), pitch = rms_sq_pitch(a.n);
#pragma unroll
      for (int k = 0; k < kNormPrefetch; ++k) {
        const int idx = tid + kThreads * k;
        if (idx < lim) terms[(idx & 7) * pitch + (idx >> 3)] = xv[k] * xv[k];
      }
      scale = rms_chain_fold<kThreads>(a.x, a.n, a.norm_eps, terms, red);
    } else {
      scale = rms_scale_block<kThreads>(a.x, a.n, a.norm_eps, terms, red);
    }
    // xn = (x * scale) * w, as the reference's rmsnorm rounds it, into LDS
    float* xs = terms + a.xs_off;
    if (pre) {
#pragma unroll
      for (int k = 0; k < kNormPrefetch; ++k) {
        const int idx = tid + kThreads * k;
        if (idx < a.n) xs[xs_index(idx)] = (xv[k] * scale) * wv[k];
      }
    } else {
      for (int idx = tid; idx < a.n; idx += kThreads)
        xs[xs_index(idx)] = (a.x[idx] * scale) * a.norm_w[idx];
    }
    __syncthreads();
    if (a.xn_out && wg == 0)
      for (int idx = tid; idx < a.n; idx += kThreads) a.xn_out[idx] = xs[xs_index(idx)];
    const LdsX xsrc{xs};
    if (first) {
      unit_terms<F, RB>(a, xsrc, terms, rows, rlane, u, raw);
      unit_passes<F, RB, PAIR>(a, xsrc, terms, r0, rows, rlane, 1);
    }
  } else {
    if (active) unit_passes<F, RB, PAIR>(a, PlainX{a.x}, terms, r0, rows, rlane, 0);
  }
  __syncthreads();
  // the row's terms in order, 16 per step, the next step's reads in flight
  for (int rr = tid; rr < rows; rr += kThreads) {
    const float* t = terms + rr * a.tpitch;  // 16-byte aligned rows
    const int full = a.terms / 16 * 16;
    float sumf = 0.0f;
    if (full > 0) {
      float4 nx[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) nx[i] = *(const float4*)(t + 4 * i);
      for (int s = 0; s < full; s += 16) {
        float4 cur[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) cur[i] = nx[i];
        if (s + 16 < full) {
#pragma unroll
          for (int i = 0; i < 4; ++i) nx[i] = *(const float4*)(t + s + 16 + 4 * i);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sumf = sumf + cur[i].x;
          sumf = sumf + cur[i].y;
          sumf = sumf + cur[i].z;
          sumf = sumf + cur[i].w;
        }
      }
    }
    for (int s = full; s < a.terms; ++s) sumf = sumf + t[s];
    const int r = r0 + rr;
    if constexpr (PAIR) {
      // rows come in (gate, up) pairs on adjacent lanes (r0 and rows even)
      const float g = __shfl_xor(sumf, 1);
      if (r & 1) a.out[r >> 1] = silu(g) * sumf;
    } else {
      if (a.bias_mode == 1) sumf = sumf + a.bias[r];
      if (a.bias_mode == 2) sumf = sumf + 0.0f;
      if (a.gate) sumf = silu(a.gate[r]) * sumf;
      if (a.resid) sumf = a.resid[r] + sumf;
      a.out[r] = sumf;
    }
  }
}

// ---- batched GEMV: matmul_batch (tensor.c:322-366) ------------------------
// out[t][i] = vec_dot(row i, x[t]) for the tokens of a prompt chunk, each
// (row, token) with exactly the single-vector kernel's arithmetic.  A
// workgroup holds its rows' weights in registers and runs up to kTokTile
// tokens over them; the token tiles of one row tile share an XCD (and its
// L2), so the weights come from HBM about once per chunk.
// Four tokens per workgroup measured fastest for a 128-token TinyLlama
// prompt (1, 2, 3, 5, 6, 8 tokens: 28.6, 21.5, 20.4, 19.2, 22.2, 20.1 ms
// against 18.3; 16 leave no room for the term buffer).
constexpr int kTokTile = 4;

struct BatchArgs {
  GemvArgs a;
  int n_tok, x_stride, out_stride;  // tokens, floats between x rows / out rows
  int row_tiles, tok_tiles;
};

template <class F, int RB, bool PAIR>
__global__ __launch_bounds__(kThreads) void gemm_kernel(BatchArgs b) {
  extern __shared__ __align__(16) float terms[];  // [row][token][tpitch]
  const GemvArgs& a = b.a;
  const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int r_tile = (k / b.tok_tiles) * 8 + xcd;
  const int t_tile = k % b.tok_tiles;
  if (r_tile >= b.row_tiles) return;
  const int tid = threadIdx.x;
  const int r0 = r_tile * a.rows_per_wg;
  const int rows = min(a.rows_per_wg, (PAIR ? 2 * a.d : a.d) - r0);
  const int tk0 = t_tile * kTokTile;
  const int toks = min(kTokTile, b.n_tok - tk0);
  const int rlane = tid / a.uspan;
  if (rlane < a.row_par) {
    for (int it = 0; it < a.unit_iters; ++it) {
      const int u = tid % a.uspan + it * a.uspan;
      if (u >= a.units) break;
      typename F::Raw raw[RB];
      load_rows<F, RB, PAIR>(a, r0, rows, rlane, u, raw);
      for (int t = 0; t < toks; ++t) {
        typename F::X U;
        F::load_x(PlainX{a.x + (size_t)(tk0 + t) * b.x_stride}, u, U);
#pragma unroll
        for (int kk = 0; kk < RB; ++kk) {
          float tt[F::kTerms];
          F::terms(u, raw[kk], U, tt);
          const int rr = rlane + a.row_par * kk;
          if (rr < rows) {
#pragma unroll
            for (int g = 0; g < F::kTerms; ++g)
              terms[(rr * kTokTile + t) * a.tpitch + F::term_index(u) + g] = tt[g];
          }
        }
      }
    }
  }
  __syncthreads();
  // one thread per (row, token): idx = t * rows + rr keeps a gate/up pair on
  // adjacent lanes (rows even)
  for (int idx = tid; idx < rows * toks; idx += kThreads) {
    const int t = idx / rows, rr = idx - t * rows;
    const float* tp = terms + (rr * kTokTile + t) * a.tpitch;
    float sumf = 0.0f;
    for (int s = 0; s < a.terms; s += 4) {
      const float4 v = *(const float4*)(tp + s);
      sumf = sumf + v.x;
      if (s + 1 < a.terms) sumf = sumf + v.y;
      if (s + 2 < a.terms) sumf = sumf + v.z;
      if (s + 3 < a.terms) sumf = sumf + v.w;
    }
    const int r = r0 + rr;
    const size_t o = (size_t)(tk0 + t) * b.out_stride;
    if constexpr (PAIR) {
      const float g = __shfl_xor(sumf, 1);
      if (r & 1) a.out[o + (r >> 1)] = silu(g) * sumf;
    } else {
      if (a.bias_mode == 1) sumf = sumf + a.bias[r];
      if (a.bias_mode == 2) sumf = sumf + 0.0f;
      if (a.gate) sumf = silu(a.gate[o + r]) * sumf;
      if (a.resid) sumf = a.resid[o + r] + sumf;
      a.out[o + r] = sumf;
    }
  }
}

template <class F, int RB, bool NORM, bool PAIR>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) float terms[];
  gemv_body<F, RB, NORM, PAIR>(a, blockIdx.x, terms);
}

// Several GEMVs over the same x in one launch (the q, k and v projections),
// each a segment of the grid with its own type, or one gate/up pair.
constexpr int kMaxSeg = 3;
struct MultiArgs {
  GemvArgs seg[kMaxSeg];
  int qtype[kMaxSeg];
  int wg0[kMaxSeg + 1];  // first workgroup of each segment, then the grid size
  int nseg;
};

template <int RB, bool NORM, bool PAIR>
__global__ __launch_bounds__(kThreads) void gemv_multi_kernel(MultiArgs m) {
  extern __shared__ __align__(16) float terms[];
  int s = 0;
  while (s + 1 < m.nseg && (int)blockIdx.x >= m.wg0[s + 1]) ++s;
  const int wg = blockIdx.x - m.wg0[s];
  switch (m.qtype[s]) {
    case kTypeQ4K: gemv_body<Q4K, RB, NORM, PAIR>(m.seg[s], wg, terms); break;
    case kTypeQ8_0: gemv_body<Q80, RB, NORM, PAIR>(m.seg[s], wg, terms); break;
    default: gemv_body<Q6K<4>, RB, NORM, PAIR>(m.seg[s], wg, terms); break;
  }
}

// ---- the fast order: x as fixed-point int8 digits, integer dot products --
//
// Within the forward pass's tolerance instead of bit-identical to the x86
// AVX2 order (plh_set_tuning key 10 selects the exact kernels above).  x, or
// rmsnorm(x) (its sum of squares reduced as a tree), is staged once per
// workgroup in LDS: each 32-element block b gets a power-of-two scale 2^-k_b
// with max|x| * 2^k_b < 2^30, and each element the integer
// X = rint(x * 2^k_b) as four signed base-256 digits X = D3 * 2^24 +
// D2 * 2^16 + D1 * 2^8 + D0 (each in [-128, 127]) in four byte planes; the
// sums of x over each 16 elements are kept in fp32.  A quad of quant values
// against a digit word is one exact v_dot4_i32_i8 per digit; per block the
// four integer sums become a float once, (S3 * 2^24 + ... + S0) * 2^-k_b.
// The roundings are that combine, the scale products, the term sums (in any
// order) and the quantization of x to 30 bits relative to its block's
// largest element (at most 2^-31 of it per element): measured on random
// blocks, ~3e-8 of sum |q x| per block, 6e-7 when one element is 1000x the
// others and meets a zero weight, 7e-6 at 1e4x.  A block spanning more
// magnitudes than that loses its small elements' precision; the exact order
// has no such limit.  About 4.5 lane instructions per Q4_K weight saved.
constexpr int kDigitBlock = 32;
constexpr int kDigits = 4;

// Word w of a digit plane (4 elements per word), padded by 4 words per 16 so
// that lanes reading adjacent 64-element units start in different banks.
__host__ __device__ inline int dg_index(int w) { return w + 4 * (w >> 4); }

struct DigitStage {  // LDS layout of the staged x, in 4-byte words
  int plane;         // words per digit plane
  int scales;        // the block scales 2^-k (float)
  int sums;          // the 16-element sums (float)
  int words;         // total
};
__host__ __device__ inline DigitStage digit_stage(int n) {
  DigitStage d;
  d.plane = (dg_index(n / 4 - 1) + 4) / 4 * 4;
  d.scales = kDigits * d.plane;
  d.sums = d.scales + n / kDigitBlock;
  d.words = d.sums + n / 16;
  return d;
}

// The staged x of a workgroup, as the digit formats read it.
struct DigLds {
  const uint32_t* base;
  DigitStage st;
};

// This thread's first 8-element chunk of x (and of the norm weights), loaded
// before the workgroup's weight loads: loads complete in issue order, so x
// loaded after them would wait for all of them and the staging below could
// not overlap the weight stream.
// Without the norm prologue the first three chunks (x up to 6144
// elements); with it the first chunk and its norm weights.
template <bool NORM>
struct XFirst {
  static constexpr int N = NORM ? 1 : 3;
  float4 x0[N], x1[N], w0, w1;
};
template <bool NORM>
__device__ __forceinline__ void load_x_first(const GemvArgs& a, XFirst<NORM>& f) {
  const int nch = a.n / 8;
  f.w0 = f.w1 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < XFirst<NORM>::N; ++j) {
    const int c = threadIdx.x + j * kThreads;
    f.x0[j] = f.x1[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c < nch) {
      f.x0[j] = ld4(a.x + 8 * c);
      f.x1[j] = ld4(a.x + 8 * c + 4);
    }
  }
  if constexpr (NORM) {
    const int c = threadIdx.x;
    if (c < nch) {
      f.w0 = ld4(a.norm_w + 8 * c);
      f.w1 = ld4(a.norm_w + 8 * c + 4);
    }
  }
}

// Stages x (NORM: rmsnorm(x, norm_w), the reference's formula with its sum
// of squares reduced as a tree) into dst.  Thread t takes the 8-element
// chunks t, t + kThreads, ...: the four chunks of a 32-element block sit on
// four adjacent lanes.  Workgroup wg 0 also stores rmsnorm(x) to xn_out.
// One 8-element chunk c of x (x0, x1; w0, w1 its norm weights for NORM)
// scaled and staged as digits.  Every lane calls it (the shuffles need all
// of them), ok false past the end of x.
template <bool NORM>
__device__ __forceinline__ void stage_chunk(const GemvArgs& a, int wg, int c, bool ok,
                                            float4 x0, float4 x1, float4 w0, float4 w1,
                                            float scale, uint32_t* dst, const DigitStage& st) {
  float v[8];
  if (ok) {
    v[0] = x0.x, v[1] = x0.y, v[2] = x0.z, v[3] = x0.w;
    v[4] = x1.x, v[5] = x1.y, v[6] = x1.z, v[7] = x1.w;
    if constexpr (NORM) {
      const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (v[j] * scale) * w[j];
      if (a.xn_out && wg == 0) {
        *(float4*)(a.xn_out + 8 * c) = make_float4(v[0], v[1], v[2], v[3]);
        *(float4*)(a.xn_out + 8 * c + 4) = make_float4(v[4], v[5], v[6], v[7]);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = 0.0f;
  }
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
  m = fmaxf(m, __shfl_xor(m, 1, 64));
  m = fmaxf(m, __shfl_xor(m, 2, 64));
  // max|x| = f * 2^e, f in [0.5, 1): 2^k = 2^(30 - e) keeps |X| < 2^30.
  // A block with an infinite or NaN element gets a NaN scale, so its
  // outputs are NaN (the reference's fp32 products would give inf or NaN).
  int k = 0;
  if (m > 0.0f && m <= 3.4028235e38f) k = 30 - __builtin_amdgcn_frexp_expf(m);
  // Balanced base-256 digits of X (|X| < 2^30): the bytes of
  // Z = (X + 0x80808080) ^ 0x80808080 read as signed bytes (byte p of
  // X + 0x80808080 is D_p + 128).  A 4 x 4 byte transpose of four elements'
  // Z then gives the digit words (word p: byte p of each element).
  uint32_t dw[kDigits][2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    uint32_t z[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int X = (int)rintf(__builtin_amdgcn_ldexpf(v[4 * q + b], k));
      z[b] = ((uint32_t)X + 0x80808080u) ^ 0x80808080u;
    }
    // perm(hi, lo, sel): byte i of the result is byte sel_i of {hi:lo}
    const uint32_t t0 = __builtin_amdgcn_perm(z[1], z[0], 0x05010400u);  // z0.0 z1.0 z0.1 z1.1
    const uint32_t t1 = __builtin_amdgcn_perm(z[1], z[0], 0x07030602u);  // z0.2 z1.2 z0.3 z1.3
    const uint32_t t2 = __builtin_amdgcn_perm(z[3], z[2], 0x05010400u);
    const uint32_t t3 = __builtin_amdgcn_perm(z[3], z[2], 0x07030602u);
    dw[0][q] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    dw[1][q] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    dw[2][q] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    dw[3][q] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
  }
  float s16 = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  s16 += __shfl_xor(s16, 1, 64);
  if (ok) {
#pragma unroll
    for (int p = 0; p < kDigits; ++p)
      *(uint2*)(dst + p * st.plane + dg_index(2 * c)) = make_uint2(dw[p][0], dw[p][1]);
    if ((c & 1) == 0) reinterpret_cast<float*>(dst)[st.sums + c / 2] = s16;
    if ((c & 3) == 0) {
      const bool fin = m <= 3.4028235e38f;
      reinterpret_cast<float*>(dst)[st.scales + c / 4] =
          fin ? __builtin_amdgcn_ldexpf(1.0f, -k) : __builtin_nanf("");
    }
  }
}

template <bool NORM>
__device__ __forceinline__ void stage_digits(const GemvArgs& a, int wg, const XFirst<NORM>& xf,
                                             uint32_t* dst, float* red) {
  const int tid = threadIdx.x;
  const int n = a.n;
  const DigitStage st = digit_stage(n);
  const int nch = n / 8;  // a multiple of 4: whole blocks
  float scale = 1.0f;
  if constexpr (NORM) {
    // sum of squares over this thread's chunks tid, tid + kThreads, ...
    float ss = 0.0f;
    if (tid < nch) {
      const float4 v = xf.x0[0], u = xf.x1[0];
      ss = ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w)) +
           ((u.x * u.x + u.y * u.y) + (u.z * u.z + u.w * u.w));
    }
    for (int c = tid + kThreads; c < nch; c += kThreads) {
      const float4 v = ld4(a.x + 8 * c), u = ld4(a.x + 8 * c + 4);
      ss += ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w)) +
            ((u.x * u.x + u.y * u.y) + (u.z * u.z + u.w * u.w));
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    scale = 1.0f / sqrtf(ss / (float)n + a.norm_eps);
  }
  // the chunks already in registers, then the rest
#pragma unroll
  for (int j = 0; j < XFirst<NORM>::N; ++j) {
    const int c0 = j * kThreads;  // uniform
    if (c0 < nch)
      stage_chunk<NORM>(a, wg, c0 + tid, c0 + tid < nch, xf.x0[j], xf.x1[j], xf.w0, xf.w1, scale,
                        dst, st);
  }
  for (int c0 = XFirst<NORM>::N * kThreads; c0 < nch; c0 += kThreads) {
    const int c = c0 + tid;
    const bool ok = c < nch;  // uniform over the four lanes of a block
    float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0, w0 = x0, w1 = x0;
    if (ok) {
      x0 = ld4(a.x + 8 * c);
      x1 = ld4(a.x + 8 * c + 4);
      if constexpr (NORM) {
        w0 = ld4(a.norm_w + 8 * c);
        w1 = ld4(a.norm_w + 8 * c + 4);
      }
    }
    stage_chunk<NORM>(a, wg, c, ok, x0, x1, w0, w1, scale, dst, st);
  }
}

// x of one unit: NW digit words per plane (4 elements each), the scales of
// its 32-element blocks and the sums of its 16-element groups.
template <int NW>
struct XDig {
  uint32_t d[kDigits][NW];
  float sc[NW / 8];
  float sx[NW / 4];
};
template <int NW>
__device__ __forceinline__ void load_xdig(const DigLds& src, int u, XDig<NW>& U) {
  const int w0 = NW * u;  // first word of the unit
#pragma unroll
  for (int p = 0; p < kDigits; ++p)
#pragma unroll
    for (int i = 0; i < NW; i += 4) {
      const uint4 v = *(const uint4*)(src.base + p * src.st.plane + dg_index(w0 + i));
      U.d[p][i] = v.x, U.d[p][i + 1] = v.y, U.d[p][i + 2] = v.z, U.d[p][i + 3] = v.w;
    }
  const float* f = reinterpret_cast<const float*>(src.base);
#pragma unroll
  for (int b = 0; b < NW / 8; ++b) U.sc[b] = f[src.st.scales + NW / 8 * u + b];
#pragma unroll
  for (int g = 0; g < NW / 4; ++g) U.sx[g] = f[src.st.sums + NW / 4 * u + g];
}

// (S3 * 2^24 + S2 * 2^16 + S1 * 2^8 + S0) of the digit sums
__device__ __forceinline__ float digit_value(const int (&s)[kDigits]) {
  return __builtin_fmaf(
      (float)s[3], 16777216.0f,
      __builtin_fmaf((float)s[2], 65536.0f, __builtin_fmaf((float)s[1], 256.0f, (float)s[0])));
}

// Q4_K: the unit is one 64-element sub-block pair (low nibbles: sub-block
// 2j, elements 0-31; high nibbles: 2j + 1, elements 32-63)
struct Q4KD : Q4K {
  using X = XDig<16>;
  template <class XS>
  static __device__ __forceinline__ void load_x(const XS& x, int u, X& U) {
    load_xdig<16>(x, u, U);
  }
  static __device__ __forceinline__ void terms(int u, const Raw& r, const X& U, float* t) {
    const int j = u & 3;
    const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    int s1[kDigits] = {}, s2[kDigits] = {};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int p = 0; p < kDigits; ++p) {
        s1[p] = __builtin_amdgcn_sdot4((int)lo, (int)U.d[p][i], s1[p], false);
        s2[p] = __builtin_amdgcn_sdot4((int)hi, (int)U.d[p][8 + i], s2[p], false);
      }
    }
    const float qx1 = digit_value(s1) * U.sc[0], qx2 = digit_value(s2) * U.sc[1];
    const float sx1 = U.sx[0] + U.sx[1], sx2 = U.sx[2] + U.sx[3];
    const float dd = f16_bits_to_f32((uint16_t)(r.hdr.x & 0xFFFFu));
    const float dmin = f16_bits_to_f32((uint16_t)(r.hdr.x >> 16));
    int sc, mn;
    scale_min(2 * j, r.hdr, sc, mn);
    const float d1 = dd * (float)sc, m1 = dmin * (float)mn;
    scale_min(2 * j + 1, r.hdr, sc, mn);
    const float d2 = dd * (float)sc, m2 = dmin * (float)mn;
    t[0] = (d1 * qx1 - m1 * sx1) + (d2 * qx2 - m2 * sx2);
  }
};

// Q6_K: the unit is four 16-element groups; value v - 32 times d * scale
struct Q6KD : Q6K<4> {
  using X = XDig<16>;
  template <class XS>
  static __device__ __forceinline__ void load_x(const XS& x, int u, X& U) {
    load_xdig<16>(x, u, U);
  }
  static __device__ __forceinline__ void terms(int, const Raw& r, const X& U, float* t) {
    const float dd = f16_bits_to_f32((uint16_t)(r.d & 0xFFFFu));
    const uint32_t m4 = 0x0F0F0F0Fu, m30 = 0x30303030u;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t L0 = r.q[0][g], L1 = r.q[1][g], H = r.q[2][g];
      const uint32_t v[4] = {(L0 & m4) | ((H << 4) & m30), ((L0 >> 4) & m4) | ((H << 2) & m30),
                             (L1 & m4) | (H & m30), ((L1 >> 4) & m4) | ((H >> 2) & m30)};
      int s[kDigits] = {};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int p = 0; p < kDigits; ++p)
          s[p] = __builtin_amdgcn_sdot4((int)v[i], (int)U.d[p][4 * g + i], s[p], false);
      const float vx = digit_value(s) * U.sc[g / 2];
      t[g] = (dd * sbyte(r.sc, g)) * (vx - 32.0f * U.sx[g]);
    }
  }
};

// Q8_0: the unit is one 32-element block of signed quants
struct Q80D : Q80 {
  using X = XDig<8>;
  template <class XS>
  static __device__ __forceinline__ void load_x(const XS& x, int u, X& U) {
    load_xdig<8>(x, u, U);
  }
  static __device__ __forceinline__ void terms(int, const Raw& r, const X& U, float* t) {
    const uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    int s[kDigits] = {};
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int p = 0; p < kDigits; ++p)
        s[p] = __builtin_amdgcn_sdot4((int)qw[i], (int)U.d[p][i], s[p], false);
    t[0] = f16_bits_to_f32((uint16_t)(r.d & 0xFFFFu)) * (digit_value(s) * U.sc[0]);
  }
};

// Unit u's terms of this thread's RB rows, added to its per-row sums.
template <class F, int RB>
__device__ __forceinline__ void unit_acc(const DigLds& xs, int u, const typename F::Raw (&raw)[RB],
                                         float (&acc)[RB]) {
  typename F::X U;
  F::load_x(xs, u, U);
#pragma unroll
  for (int k = 0; k < RB; ++k) {
    float t[F::kTerms];
    F::terms(u, raw[k], U, t);
    float s = t[0];
#pragma unroll
    for (int g = 1; g < F::kTerms; ++g) s += t[g];
    acc[k] += s;
  }
}

// One workgroup of the fast order: rows [r0, r0 + rows_per_wg).  The first
// pass's weight loads are issued, x is staged as digits (after rmsnorm for
// NORM), then each thread adds its units' terms per row in registers (later
// passes load and add more units); the uspan sums of a row go through LDS
// and are added by a power-of-two group of lanes (a shuffle tree), which
// applies the epilogue.
// COH: the outputs are read by other workgroups of the same launch (the fused
// q/k/v + attention launch): stored at device scope.
template <class F, int RB, bool NORM, bool PAIR, bool COH = false>
__device__ __forceinline__ void gemv_body_fast(const GemvArgs& a, int wg, float* lds) {
  __shared__ float red[kThreads / 64];
  const int tid = threadIdx.x;
  const int r0 = wg * a.rows_per_wg;
  const int rows = min(a.rows_per_wg, (PAIR ? 2 * a.d : a.d) - r0);
  const int rlane = tid / a.uspan;
  const bool active = rlane < a.row_par;
  const int u = tid % a.uspan;
  const bool first = active && u < a.units;
  XFirst<NORM> xf;
  load_x_first<NORM>(a, xf);
  // A gate/up pair issues one row's weights before staging x and the rest
  // after it: the issue of a workgroup's whole weight block can stall on
  // the CU's outstanding requests and hold the staging back (measured on the
  // TinyLlama pair, 8.3 -> 7.9 us; single GEMVs measured better with every
  // row issued first).
  typename F::Raw raw[RB];
  if constexpr (PAIR) {
    if (first) load_rows_k<F, RB, PAIR, 0, 1>(a, r0, rows, rlane, u, raw);
  } else {
    if (first) load_rows<F, RB, PAIR>(a, r0, rows, rlane, u, raw);
  }
  uint32_t* xd = reinterpret_cast<uint32_t*>(lds + a.xs_off);
  stage_digits<NORM>(a, wg, xf, xd, red);
  if constexpr (PAIR) {
    if (first) load_rows_k<F, RB, PAIR, 1, RB>(a, r0, rows, rlane, u, raw);
  }
  __syncthreads();
  const DigLds src{xd, digit_stage(a.n)};
  float acc[RB];
#pragma unroll
  for (int k = 0; k < RB; ++k) acc[k] = 0.0f;
  if (first) {
    unit_acc<F, RB>(src, u, raw, acc);
    for (int it = 1; it < a.unit_iters; ++it) {
      const int uu = u + it * a.uspan;
      if (uu >= a.units) break;
      load_rows<F, RB, PAIR>(a, r0, rows, rlane, uu, raw);
      unit_acc<F, RB>(src, uu, raw, acc);
    }
  }
  // row rr's per-thread sums at lds[rr * uspan + u] (the term buffer's space)
  if (first) {
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      const int rr = rlane + a.row_par * k;
      if (rr < rows) lds[rr * a.uspan + u] = acc[k];
    }
  }
  __syncthreads();
  // tpr lanes per row (a power of two, at most 32 so that a gate/up pair's
  // two rows share a wave)
  int tpr = 1;
  while (tpr < 32 && 2 * tpr * a.rows_per_wg <= kThreads) tpr *= 2;
  const int j = tid & (tpr - 1);
  const int nsum = min(a.units, a.uspan);
  for (int rr0 = 0; rr0 < rows; rr0 += kThreads / tpr) {
    const int rr = rr0 + tid / tpr;  // uniform over the tpr lanes
    float sumf = 0.0f;
    if (rr < rows)
      for (int i = j; i < nsum; i += tpr) sumf += lds[rr * a.uspan + i];
    for (int m = tpr / 2; m >= 1; m >>= 1) sumf += __shfl_xor(sumf, m, 64);
    const int r = r0 + rr;
    if constexpr (PAIR) {
      const float g = __shfl_xor(sumf, tpr, 64);  // the gate row's sum
      if (rr < rows && j == 0 && (r & 1)) a.out[r >> 1] = silu(g) * sumf;
    } else {
      if (rr < rows && j == 0) {
        if (a.bias_mode == 1) sumf = sumf + a.bias[r];
        if (a.bias_mode == 2) sumf = sumf + 0.0f;
        if (a.gate) sumf = silu(a.gate[r]) * sumf;
        if (a.resid) sumf = a.resid[r] + sumf;
        if constexpr (COH)
          __hip_atomic_store(a.out + r, sumf, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          a.out[r] = sumf;
      }
    }
  }
}

template <class F, int RB, bool NORM, bool PAIR>
__global__ __launch_bounds__(kThreads) void gemv_fast_kernel(GemvArgs a) {
  extern __shared__ __align__(16) float terms[];
  gemv_body_fast<F, RB, NORM, PAIR>(a, blockIdx.x, terms);
}

template <int RB, bool NORM>
__global__ __launch_bounds__(kThreads) void gemv_fast_multi_kernel(MultiArgs m) {
  extern __shared__ __align__(16) float terms[];
  static_assert(kMaxSeg == 3, "the segment choice below covers three segments");
  // the segment from one batch of argument loads (a search loop would chain
  // one memory round trip per step)
  PLH_ARGS_NOW("s"(m.nseg), "s"(m.wg0[1]), "s"(m.wg0[2]), "s"(m.qtype[0]), "s"(m.qtype[1]),
               "s"(m.qtype[2]));
  const int b = blockIdx.x;
  const int s = (m.nseg > 1 && b >= m.wg0[1]) + (m.nseg > 2 && b >= m.wg0[2]);
  const int wg = b - (s == 2 ? m.wg0[2] : s == 1 ? m.wg0[1] : 0);
  const int qtype = s == 2 ? m.qtype[2] : s == 1 ? m.qtype[1] : m.qtype[0];
  // the segment's arguments: a second (and last) batch
  const GemvArgs& g = m.seg[s];
  PLH_ARGS_NOW("s"(g.w), "s"(g.x), "s"(g.out), "s"(g.d), "s"(g.nb), "s"(g.units), "s"(g.uspan),
               "s"(g.row_par), "s"(g.unit_iters), "s"(g.rows_per_wg), "s"(g.off0), "s"(g.off1),
               "s"(g.off2), "s"(g.scales_off), "s"(g.d_off), "s"(g.n), "s"(g.xs_off),
               "s"(g.bias), "s"(g.gate), "s"(g.resid), "s"(g.bias_mode), "s"(g.norm_w),
               "s"(g.norm_eps), "s"(g.xn_out));
  switch (qtype) {
    case kTypeQ4K: gemv_body_fast<Q4KD, RB, NORM, false>(m.seg[s], wg, terms); break;
    case kTypeQ8_0: gemv_body_fast<Q80D, RB, NORM, false>(m.seg[s], wg, terms); break;
    default: gemv_body_fast<Q6KD, RB, NORM, false>(m.seg[s], wg, terms); break;
  }
}

// ---- q/k/v projections and the attention in one launch (plh_forward) ------
//
// Workgroups 0 .. n_att - 1 are the layer's attention (one unsplit group
// each, attn_decode_body's fused form); the rest are gemv_fast_multi_kernel's
// q, k and v workgroups, which store their rows at device scope and then
// count themselves in on the counter of every group their rows belong to.
// The attention workgroups issue their first cached tiles, wait for their
// group's count, and go on as the split kernel does: one launch instead of
// two, and the attention's cache loads overlap the projections.
struct FusedArgs {
  MultiArgs m;   // q, k, v (segments 0, 1, 2); wg0 counts from workgroup n_att
  DecodeArgs d;  // the layer's unsplit attention
  FuseWait fw;
  int n_att;
  PfLaunch pl;   // workgroups pl.n_main.. prefetch the next GEMVs' weights
};

template <int D, int RB>
__global__ __launch_bounds__(kThreads) void qkv_attn_fused_kernel(FusedArgs f) {
  extern __shared__ __align__(16) float terms[];
  static_assert(64 * DecodeShape<D>::W == kThreads, "one workgroup shape for both roles");
  if ((int)blockIdx.x < f.n_att) {
    attn_decode_body<D, false, false, true>(f.d, PfLaunch{}, f.fw);
    return;
  }
  const MultiArgs& m = f.m;
  PLH_ARGS_NOW("s"(f.n_att), "s"(m.wg0[1]), "s"(m.wg0[2]), "s"(m.qtype[0]), "s"(m.qtype[1]),
               "s"(m.qtype[2]), "s"(f.pl.n_main));
  if (l2_prefetch_role(f.pl.plan, f.pl.n_main, kThreads / 64, terms)) return;
  const int b = (int)blockIdx.x - f.n_att;
  const int s = (b >= m.wg0[1]) + (b >= m.wg0[2]);
  const int wg = b - (s == 2 ? m.wg0[2] : s == 1 ? m.wg0[1] : 0);
  const int qtype = s == 2 ? m.qtype[2] : s == 1 ? m.qtype[1] : m.qtype[0];
  const GemvArgs& g = m.seg[s];
  PLH_ARGS_NOW("s"(g.w), "s"(g.x), "s"(g.out), "s"(g.d), "s"(g.nb), "s"(g.units), "s"(g.uspan),
               "s"(g.row_par), "s"(g.unit_iters), "s"(g.rows_per_wg), "s"(g.off0), "s"(g.off1),
               "s"(g.off2), "s"(g.scales_off), "s"(g.d_off), "s"(g.n), "s"(g.xs_off),
               "s"(g.bias), "s"(g.bias_mode), "s"(g.norm_w), "s"(g.norm_eps));
  switch (qtype) {
    case kTypeQ4K: gemv_body_fast<Q4KD, RB, true, false, true>(g, wg, terms); break;
    case kTypeQ8_0: gemv_body_fast<Q80D, RB, true, false, true>(g, wg, terms); break;
    default: gemv_body_fast<Q6KD, RB, true, false, true>(g, wg, terms); break;
  }
  // every row stored before the counts go up
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int r0 = wg * g.rows_per_wg;
    const int r1 = min(r0 + g.rows_per_wg, g.d);
    const int per = f.fw.group_rows[s];
    for (int grp = r0 / per; grp <= (r1 - 1) / per; ++grp)
      __hip_atomic_fetch_add(f.fw.ctr + grp * kFuseCtrPitch, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <class F, bool NORM, bool PAIR>
void launch_rb(int rb, int grid, size_t lds, hipStream_t st, const GemvArgs& a) {
  switch (rb) {
    case 1:
      hipLaunchKernelGGL((gemv_kernel<F, 1, NORM, PAIR>), dim3(grid), dim3(kThreads), lds, st, a);
      break;
    case 2:
      hipLaunchKernelGGL((gemv_kernel<F, 2, NORM, PAIR>), dim3(grid), dim3(kThreads), lds, st, a);
      break;
    case 4:
      hipLaunchKernelGGL((gemv_kernel<F, 4, NORM, PAIR>), dim3(grid), dim3(kThreads), lds, st, a);
      break;
    default:
      hipLaunchKernelGGL((gemv_kernel<F, 8, NORM, PAIR>), dim3(grid), dim3(kThreads), lds, st, a);
      break;
  }
}

template <class F>
void launch_fmt(bool norm, bool pair, int rb, int grid, size_t lds, hipStream_t st,
                const GemvArgs& a) {
  if (pair && norm)
    launch_rb<F, true, true>(rb, grid, lds, st, a);
  else if (pair)
    launch_rb<F, false, true>(rb, grid, lds, st, a);
  else if (norm)
    launch_rb<F, true, false>(rb, grid, lds, st, a);
  else
    launch_rb<F, false, false>(rb, grid, lds, st, a);
}

template <class F, bool NORM, bool PAIR>
void launch_rb_fast(int rb, int grid, size_t lds, hipStream_t st, const GemvArgs& a) {
  switch (rb) {
    case 1:
      hipLaunchKernelGGL((gemv_fast_kernel<F, 1, NORM, PAIR>), dim3(grid), dim3(kThreads), lds, st,
                         a);
      break;
    case 2:
      hipLaunchKernelGGL((gemv_fast_kernel<F, 2, NORM, PAIR>), dim3(grid), dim3(kThreads), lds, st,
                         a);
      break;
    case 4:
      hipLaunchKernelGGL((gemv_fast_kernel<F, 4, NORM, PAIR>), dim3(grid), dim3(kThreads), lds, st,
                         a);
      break;
    default:
      hipLaunchKernelGGL((gemv_fast_kernel<F, 8, NORM, PAIR>), dim3(grid), dim3(kThreads), lds, st,
                         a);
      break;
  }
}

template <class F>
void launch_fmt_fast(bool norm, bool pair, int rb, int grid, size_t lds, hipStream_t st,
                     const GemvArgs& a) {
  if (pair && norm)
    launch_rb_fast<F, true, true>(rb, grid, lds, st, a);
  else if (pair)
    launch_rb_fast<F, false, true>(rb, grid, lds, st, a);
  else if (norm)
    launch_rb_fast<F, true, false>(rb, grid, lds, st, a);
  else
    launch_rb_fast<F, false, false>(rb, grid, lds, st, a);
}

template <bool NORM>
void launch_multi_fast(int rb, int grid, size_t lds, hipStream_t st, const MultiArgs& m) {
  switch (rb) {
    case 1:
      hipLaunchKernelGGL((gemv_fast_multi_kernel<1, NORM>), dim3(grid), dim3(kThreads), lds, st,
                         m);
      break;
    case 2:
      hipLaunchKernelGGL((gemv_fast_multi_kernel<2, NORM>), dim3(grid), dim3(kThreads), lds, st,
                         m);
      break;
    default:
      hipLaunchKernelGGL((gemv_fast_multi_kernel<4, NORM>), dim3(grid), dim3(kThreads), lds, st,
                         m);
      break;
  }
}

template <bool NORM>
void launch_multi(int rb, int grid, size_t lds, hipStream_t st, const MultiArgs& m) {
  switch (rb) {
    case 1:
      hipLaunchKernelGGL((gemv_multi_kernel<1, NORM, false>), dim3(grid), dim3(kThreads), lds, st,
                         m);
      break;
    case 2:
      hipLaunchKernelGGL((gemv_multi_kernel<2, NORM, false>), dim3(grid), dim3(kThreads), lds, st,
                         m);
      break;
    default:
      hipLaunchKernelGGL((gemv_multi_kernel<4, NORM, false>), dim3(grid), dim3(kThreads), lds, st,
                         m);
      break;
  }
}

// Fills everything of a but rows_per_wg from one call.  0 or -1 (error set).
int prepare(const GemvCall& g, GemvArgs& a) {
  Layout L;
  if (!make_layout(g.qtype, g.n, g.d, L)) {
    set_error("plh_gemv: no GEMV for type %d with n=%d d=%d", g.qtype, g.n, g.d);
    return -1;
  }
  if (!g.w || !g.x || !g.out) {
    set_error("plh_gemv: null pointer");
    return -1;
  }
  if (g.bias && g.bias_zero) {
    set_error("plh_gemv_ex: a bias and bias_zero together");
    return -1;
  }
  if (g.norm_w && g.n > kMaxNormN) {
    set_error("plh_gemv_ex: rmsnorm of %d elements exceeds %d", g.n, kMaxNormN);
    return -1;
  }
  const int n = g.n, qtype = g.qtype;
  a = GemvArgs{};
  a.w = (const uint8_t*)g.w;
  a.x = g.x;
  a.out = g.out;
  a.d = g.d;
  a.nb = L.nb;
  // Q6_K lanes take four groups (64 weights, like a Q4_K sub-block): the
  // per-row work of a unit (scale, hsum, addressing) is shared by more weights
  const int q6_groups = 4;
  a.units = qtype == kTypeQ4K ? n / 64 : (qtype == kTypeQ6K ? n / (16 * q6_groups) : n / 32);
  a.terms = qtype == kTypeQ4K ? n / 64 : (qtype == kTypeQ6K ? n / 16 : n / 32);
  a.uspan = a.units < kThreads ? a.units : kThreads;
  a.row_par = kThreads / a.uspan;
  a.unit_iters = (a.units + a.uspan - 1) / a.uspan;
  a.tpitch = (a.terms + 3) / 4 * 4 + 4;  // 16-byte rows, staggered banks
  a.off0 = (uint32_t)L.off[0];
  a.off1 = (uint32_t)L.off[1];
  a.off2 = (uint32_t)L.off[2];
  a.scales_off = (uint32_t)L.scales_off;
  a.d_off = (uint32_t)L.d_off;
  a.bias = g.bias;
  a.gate = g.gate;
  a.resid = g.resid;
  a.bias_mode = g.bias ? 1 : (g.bias_zero ? 2 : 0);
  a.norm_w = g.norm_w;
  a.norm_eps = g.norm_eps;
  a.n = n;
  a.xn_out = g.norm_w ? g.xn_out : nullptr;
  return 0;
}

int lds_rows(const GemvArgs& a) { return (int)((64 * 1024) / (sizeof(float) * (size_t)a.tpitch)); }

// Rows per thread for a launch over these segments (rows[s]: the segment's
// rows, 2d for a gate/up pair): the largest of 4, 2, 1 that still gives at
// least 0.6 workgroups per CU and keeps every workgroup's terms within 64 KiB
// of LDS (measured on the TinyLlama and output-projection shapes: more rows
// in flight per thread beat more workgroups until the grid no longer covers
// the CUs; 8 rows cost occupancy).  A pair needs an even row count per
// workgroup.  -1 when a row is too long for the term buffer.
int pick_rb(const GemvArgs* seg, const int* rows, int nseg, bool pair, int max_rb) {
  const int cus = ctx().num_cus > 0 ? ctx().num_cus : 256;
  auto grid_of = [&](int rb) {
    long g = 0;
    for (int s = 0; s < nseg; ++s) g += (rows[s] + seg[s].row_par * rb - 1) / (seg[s].row_par * rb);
    return g;
  };
  auto lds_ok = [&](int rb) {
    for (int s = 0; s < nseg; ++s)
      if (seg[s].row_par * rb > lds_rows(seg[s])) return false;
    return true;
  };
  int rb = 4;
  if (g_gemv_exact) {
    while (rb > 1 && (grid_of(rb) * 10 < 6L * cus || !lds_ok(rb))) rb /= 2;
    // with the rmsnorm prologue every workgroup pays the norm's latency, and
    // workgroups sharing a CU measured to pay it one after the other: 8 rows
    // per thread when 4 would need more than one workgroup per CU
    if (seg[0].norm_w && rb == 4 && max_rb >= 8 && grid_of(4) > cus && lds_ok(8)) rb = 8;
  } else {
    // the fast order: the most rows per thread that still leaves ~2.5
    // workgroups per CU, fewer when x is long (every workgroup stages all of
    // x): swept on the TinyLlama shapes with cold weights, the best were
    // gate/up pair 2, output projection 4, down projection (n 5632) 4, q and
    // o 1; else 1
    const double per_cu = fmin(2.5, fmax(1.0, 2.5 * 2048.0 / (double)seg[0].n));
    const long target = (long)(per_cu * cus + 0.5);
    rb = 1;
    for (int c = max_rb; c >= 1; c /= 2)
      if (grid_of(c) >= target && lds_ok(c)) {
        rb = c;
        break;
      }
  }
  if (g_gemv_rows_per_thread > 0) rb = g_gemv_rows_per_thread;
  if (rb > max_rb) rb = max_rb;
  if (pair && (seg[0].row_par * rb) % 2) rb *= 2;
  if (!lds_ok(rb)) {
    set_error("plh_gemv: row of %d weights too long for the term buffer", seg[0].n);
    return -1;
  }
  return rb;
}

// LDS of a launch, and the staged x's offset: the terms, which reuse the
// rmsnorm squares' space, then rmsnorm(x).
size_t lds_bytes(GemvArgs& a) {
  size_t lds = sizeof(float) * (size_t)a.rows_per_wg * a.tpitch;
  a.xs_off = 0;
  if (a.norm_w) {
    const size_t sq = sizeof(float) * 8 * (size_t)rms_sq_pitch(a.n);
    if (sq > lds) lds = sq;
    lds = (lds + 15) / 16 * 16;
    a.xs_off = (int)(lds / sizeof(float));
    lds += sizeof(float) * (size_t)xs_floats(a.n);
  }
  return lds;
}

// LDS of a fast-order launch: the terms, then x's digits.
size_t lds_bytes_fast(GemvArgs& a) {
  size_t lds = sizeof(float) * (size_t)a.rows_per_wg * a.tpitch;
  lds = (lds + 15) / 16 * 16;
  a.xs_off = (int)(lds / sizeof(float));
  return lds + sizeof(uint32_t) * (size_t)digit_stage(a.n).words;
}

int launch_single(int qtype, bool pair, const GemvArgs& a0, int rows) {
  GemvArgs a = a0;
  const int rb = pick_rb(&a, &rows, 1, pair, 8);
  if (rb < 0) return -1;
  a.rows_per_wg = a.row_par * rb;
  const int grid = (rows + a.rows_per_wg - 1) / a.rows_per_wg;
  hipStream_t st = ctx().stream;
  const bool norm = a.norm_w != nullptr;
  if (!g_gemv_exact) {
    const size_t lds = lds_bytes_fast(a);
    if (qtype == kTypeQ4K)
      launch_fmt_fast<Q4KD>(norm, pair, rb, grid, lds, st, a);
    else if (qtype == kTypeQ8_0)
      launch_fmt_fast<Q80D>(norm, pair, rb, grid, lds, st, a);
    else
      launch_fmt_fast<Q6KD>(norm, pair, rb, grid, lds, st, a);
    return check_hip(hipGetLastError(), "gemv_fast_kernel launch");
  }
  const size_t lds = lds_bytes(a);
  if (qtype == kTypeQ4K)
    launch_fmt<Q4K>(norm, pair, rb, grid, lds, st, a);
  else if (qtype == kTypeQ8_0)
    launch_fmt<Q80>(norm, pair, rb, grid, lds, st, a);
  else
    launch_fmt<Q6K<4>>(norm, pair, rb, grid, lds, st, a);
  return check_hip(hipGetLastError(), "gemv_kernel launch");
}

template <class F, bool PAIR>
void launch_batch(int rb, int grid, size_t lds, hipStream_t st, const BatchArgs& b) {
  switch (rb) {
    case 1:
      hipLaunchKernelGGL((gemm_kernel<F, 1, PAIR>), dim3(grid), dim3(kThreads), lds, st, b);
      break;
    case 2:
      hipLaunchKernelGGL((gemm_kernel<F, 2, PAIR>), dim3(grid), dim3(kThreads), lds, st, b);
      break;
    default:
      hipLaunchKernelGGL((gemm_kernel<F, 4, PAIR>), dim3(grid), dim3(kThreads), lds, st, b);
      break;
  }
}

// Batched launch over n_tok tokens (x rows x_stride apart, out rows
// out_stride apart; gate and resid indexed like out).  No rmsnorm prologue.
int launch_batched(int qtype, bool pair, const GemvArgs& a0, int rows, int n_tok, int x_stride,
                   int out_stride) {
  if (a0.norm_w) {
    set_error("batched GEMV: no rmsnorm prologue (normalise the rows first)");
    return -1;
  }
  BatchArgs b{};
  b.a = a0;
  // rows per thread: the most (4, 2, 1) whose term buffer for kTokTile tokens
  // fits 64 KiB of LDS
  int rb = 4;
  while (rb > 1 &&
         (size_t)b.a.row_par * rb * kTokTile * b.a.tpitch * sizeof(float) > 64 * 1024)
    rb /= 2;
  if (pair && (b.a.row_par * rb) % 2) rb *= 2;
  const size_t lds = (size_t)b.a.row_par * rb * kTokTile * b.a.tpitch * sizeof(float);
  if (lds > 64 * 1024) {
    set_error("batched GEMV: row of %d weights too long for the term buffer", b.a.n);
    return -1;
  }
  b.a.rows_per_wg = b.a.row_par * rb;
  b.n_tok = n_tok;
  b.x_stride = x_stride;
  b.out_stride = out_stride;
  b.row_tiles = (rows + b.a.rows_per_wg - 1) / b.a.rows_per_wg;
  b.tok_tiles = (n_tok + kTokTile - 1) / kTokTile;
  const int grid = 8 * ((b.row_tiles + 7) / 8) * b.tok_tiles;
  hipStream_t st = ctx().stream;
  if (qtype == kTypeQ4K)
    pair ? launch_batch<Q4K, true>(rb, grid, lds, st, b) : launch_batch<Q4K, false>(rb, grid, lds, st, b);
  else if (qtype == kTypeQ8_0)
    pair ? launch_batch<Q80, true>(rb, grid, lds, st, b) : launch_batch<Q80, false>(rb, grid, lds, st, b);
  else
    pair ? launch_batch<Q6K<4>, true>(rb, grid, lds, st, b)
         : launch_batch<Q6K<4>, false>(rb, grid, lds, st, b);
  return check_hip(hipGetLastError(), "gemm_kernel launch");
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

int plh_matmul_batch(int qtype, int n, int d, const void* dev, const float* x, int n_batch,
                     float* out) {
  if (n_batch < 1) {
    set_error("plh_matmul_batch: n_batch %d", n_batch);
    return -1;
  }
  GemvCall g{};
  g.qtype = qtype, g.n = n, g.d = d, g.w = dev, g.x = x, g.out = out;
  g.n_tok = n_batch, g.x_stride = n, g.out_stride = d;
  if (n_batch == 1) g.n_tok = 0;
  return gemv_launch(g);
}

int plh_gemv(int qtype, int n, int d, const void* dev, const float* x, float* out) {
  return plh_gemv_ex(qtype, n, d, dev, x, out, nullptr, 0.0f, nullptr, 0, nullptr, nullptr);
}

int plh_gemv_swiglu(int qtype, int n, int d, const void* gate_dev, const void* up_dev,
                    const float* x, float* out, const float* norm_w, float norm_eps) {
  GemvCall g{}, u{};
  g.qtype = qtype, g.n = n, g.d = d, g.w = gate_dev, g.x = x, g.out = out;
  g.norm_w = norm_w, g.norm_eps = norm_eps;
  u = g;
  u.w = up_dev;
  if (!up_dev) {
    set_error("plh_gemv: null pointer");
    return -1;
  }
  return gemv_pair_launch(g, u);
}

int plh_gemv_ex(int qtype, int n, int d, const void* dev, const float* x, float* out,
                const float* norm_w, float norm_eps, const float* bias, int bias_zero,
                const float* gate, const float* resid) {
  GemvCall g{};
  g.qtype = qtype, g.n = n, g.d = d, g.w = dev, g.x = x, g.out = out;
  g.norm_w = norm_w, g.norm_eps = norm_eps, g.bias = bias, g.bias_zero = bias_zero;
  g.gate = gate, g.resid = resid;
  return gemv_launch(g);
}

}  // extern "C"

namespace plh {

int gemv_launch(const GemvCall& g) {
  if (!ctx().stream) {
    set_error("plh_gemv: plh_init has not been called");
    return -1;
  }
  GemvArgs a;
  if (prepare(g, a)) return -1;
  if (g.n_tok > 1)
    return launch_batched(g.qtype, false, a, g.d, g.n_tok, g.x_stride, g.out_stride);
  return launch_single(g.qtype, false, a, g.d);
}

int gemv_multi_launch(const GemvCall* g, int n) {
  if (!ctx().stream) {
    set_error("plh_gemv: plh_init has not been called");
    return -1;
  }
  if (n < 1 || n > kMaxSeg) {
    set_error("gemv_multi_launch: %d segments (1..%d)", n, kMaxSeg);
    return -1;
  }
  MultiArgs m{};
  int rows[kMaxSeg];
  for (int s = 0; s < n; ++s) {
    if (g[s].x != g[0].x || (g[s].norm_w == nullptr) != (g[0].norm_w == nullptr)) {
      set_error("gemv_multi_launch: segments must share x and the rmsnorm prologue");
      return -1;
    }
    if (prepare(g[s], m.seg[s])) return -1;
    m.qtype[s] = g[s].qtype;
    rows[s] = g[s].d;
  }
  const int rb = pick_rb(m.seg, rows, n, false, 4);
  if (rb < 0) return -1;
  size_t lds = 0;
  m.nseg = n;
  m.wg0[0] = 0;
  for (int s = 0; s < n; ++s) {
    m.seg[s].rows_per_wg = m.seg[s].row_par * rb;
    m.wg0[s + 1] = m.wg0[s] + (rows[s] + m.seg[s].rows_per_wg - 1) / m.seg[s].rows_per_wg;
    const size_t b = g_gemv_exact ? lds_bytes(m.seg[s]) : lds_bytes_fast(m.seg[s]);
    if (b > lds) lds = b;
  }
  if (!g_gemv_exact) {
    if (g[0].norm_w)
      launch_multi_fast<true>(rb, m.wg0[n], lds, ctx().stream, m);
    else
      launch_multi_fast<false>(rb, m.wg0[n], lds, ctx().stream, m);
    return check_hip(hipGetLastError(), "gemv_fast_multi_kernel launch");
  }
  if (g[0].norm_w)
    launch_multi<true>(rb, m.wg0[n], lds, ctx().stream, m);
  else
    launch_multi<false>(rb, m.wg0[n], lds, ctx().stream, m);
  return check_hip(hipGetLastError(), "gemv_multi_kernel launch");
}

int qkv_attention_launch(const GemvCall* g, const DecodeArgs& d, int head_dim, unsigned* ctr,
                         const PfPlan& pf, int pf_per_xcd) {
  if (!ctx().stream) {
    set_error("plh_gemv: plh_init has not been called");
    return -1;
  }
  if (g_gemv_exact || (head_dim != 64 && head_dim != 128) || !g[0].norm_w || !ctr) {
    set_error("qkv_attention_launch: needs the fast GEMV order, the rmsnorm prologue and "
              "head_dim 64 or 128");
    return -1;
  }
  MultiArgs m{};
  int rows[kMaxSeg];
  for (int s = 0; s < kMaxSeg; ++s) {
    if (g[s].x != g[0].x || g[s].norm_w != g[0].norm_w || g[s].n_tok > 1) {
      set_error("qkv_attention_launch: segments must share x and the rmsnorm prologue");
      return -1;
    }
    if (prepare(g[s], m.seg[s])) return -1;
    m.qtype[s] = g[s].qtype;
    rows[s] = g[s].d;
  }
  // the rows per thread gemv_multi_launch would pick, so the projections
  // are the same sums
  const int rb = pick_rb(m.seg, rows, kMaxSeg, false, 4);
  if (rb < 0) return -1;
  size_t lds = 0;
  m.nseg = kMaxSeg;
  m.wg0[0] = 0;
  FusedArgs f{};
  for (int s = 0; s < kMaxSeg; ++s) {
    m.seg[s].rows_per_wg = m.seg[s].row_par * rb;
    m.wg0[s + 1] = m.wg0[s] + (rows[s] + m.seg[s].rows_per_wg - 1) / m.seg[s].rows_per_wg;
    const size_t b = lds_bytes_fast(m.seg[s]);
    if (b > lds) lds = b;
    f.fw.wg_rows[s] = m.seg[s].rows_per_wg;
  }
  f.m = m;
  f.d = d;
  f.fw.ctr = ctr;
  f.fw.group_rows[0] = d.G * head_dim;  // q rows of one kv head's q heads
  f.fw.group_rows[1] = head_dim;        // k rows of one kv head
  f.fw.group_rows[2] = head_dim;
  f.n_att = d.n_units;
  f.pl.n_main = f.n_att + m.wg0[kMaxSeg];
  f.pl.plan = pf;
  f.pl.plan.per_xcd = pf_per_xcd;
  if (g_xcd_ok[ctx().device] != 1 || pf_per_xcd <= 0) f.pl.plan.n = 0;
  const int n_pf = f.pl.plan.n > 0 ? 8 * pf_per_xcd : 0;
  if (n_pf && lds < (size_t)kPfLdsBytes) lds = kPfLdsBytes;
  const dim3 grid((unsigned)(f.pl.n_main + n_pf)), block(kThreads);
  hipStream_t st = ctx().stream;
#define PLH_FUSED(D, RB) \
  hipLaunchKernelGGL((qkv_attn_fused_kernel<D, RB>), grid, block, lds, st, f)
  if (head_dim == 64) {
    if (rb == 1) PLH_FUSED(64, 1); else if (rb == 2) PLH_FUSED(64, 2); else PLH_FUSED(64, 4);
  } else {
    if (rb == 1) PLH_FUSED(128, 1); else if (rb == 2) PLH_FUSED(128, 2); else PLH_FUSED(128, 4);
  }
#undef PLH_FUSED
  return check_hip(hipGetLastError(), "qkv_attn_fused_kernel launch");
}

int gemv_pair_launch(const GemvCall& gate, const GemvCall& up) {
  if (!ctx().stream) {
    set_error("plh_gemv: plh_init has not been called");
    return -1;
  }
  if (gate.qtype != up.qtype || gate.n != up.n || gate.d != up.d || gate.x != up.x ||
      gate.norm_w != up.norm_w || gate.norm_eps != up.norm_eps || gate.bias ||
      up.bias || gate.bias_zero || up.bias_zero || gate.gate || up.gate || gate.resid ||
      up.resid) {
    set_error("gemv_pair_launch: gate and up must match in type, shape, x and rmsnorm, "
              "without other epilogues");
    return -1;
  }
  GemvArgs a;
  if (prepare(up, a)) return -1;
  a.w = (const uint8_t*)gate.w;
  a.w2 = (const uint8_t*)up.w;
  if (!a.w) {
    set_error("plh_gemv: null pointer");
    return -1;
  }
  if (up.n_tok > 1)
    return launch_batched(up.qtype, true, a, 2 * up.d, up.n_tok, up.x_stride, up.out_stride);
  return launch_single(up.qtype, true, a, 2 * up.d);
}

// Appends the plane streams of one matrix, read wg_rows rows per workgroup
// by workgroups wg0, wg0 + 1, ...; planes whose chunks are not whole 16-byte
// units are left out.
static int prefetch_matrix(int qtype, int n, int d, const void* w, int wg_rows, int wg0,
                           PfPlan& pf) {
  Layout L;
  if (!w || !make_layout(qtype, n, d, L)) return -1;
  // per-row bytes of each plane (the packed layouts of make_layout)
  const size_t nb = (size_t)L.nb;
  size_t off[5], bpr[5];
  int np = 0;
  if (qtype == kTypeQ4K) {
    off[0] = L.off[0], bpr[0] = nb * 16;
    off[1] = L.off[1], bpr[1] = nb * 64;
    off[2] = L.off[2], bpr[2] = nb * 64;
    np = 3;
  } else if (qtype == kTypeQ6K) {
    for (int p = 0; p < 3; ++p) off[p] = L.off[p], bpr[p] = nb * 64;
    off[3] = L.scales_off, bpr[3] = nb * 16;
    off[4] = L.d_off, bpr[4] = nb * 2;
    np = 5;
  } else {
    off[0] = L.off[0], bpr[0] = nb * 16;
    off[1] = L.off[1], bpr[1] = nb * 16;
    off[2] = L.d_off, bpr[2] = nb * 2;
    np = 3;
  }
  if (pf.n + np > kPfStreams) return -1;
  for (int p = 0; p < np; ++p)
    if (make_pf_stream((const uint8_t*)w + off[p], bpr[p] * (size_t)wg_rows, bpr[p] * (size_t)d,
                       wg0, pf.s[pf.n]))
      ++pf.n;
  return 0;
}

int gemv_prefetch_plan(const GemvCall& g, const GemvCall* up, PfPlan& pf) {
  GemvArgs a;
  if (g.n_tok > 1 || prepare(g, a)) return -1;
  // the rows per workgroup launch_single picks for this call
  const bool pair = up != nullptr;
  const int rows = pair ? 2 * g.d : g.d;
  const int rb = pick_rb(&a, &rows, 1, pair, 8);
  if (rb < 0) return -1;
  const int wg_rows = pair ? a.row_par * rb / 2 : a.row_par * rb;  // matrix rows
  if (prefetch_matrix(g.qtype, g.n, g.d, g.w, wg_rows, 0, pf)) return -1;
  return pair ? prefetch_matrix(up->qtype, up->n, up->d, up->w, wg_rows, 0, pf) : 0;
}

}  // namespace plh
