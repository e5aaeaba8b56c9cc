// attn_decode_dev.h -- the decode kernels' device code shared by the launch
// files: workgroup shapes, the q / new-row / tile loads, the tile product and
// the split kernel's body (attn_decode_body).  attn_decode.hip wraps it in
// its kernels; gemv.hip's fused q/k/v + attention launch of plh_forward runs
// the body in its attention workgroups.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_common.h"
#include "picolm_hip.h"
#include "plh_internal.h"

namespace {
using namespace plh;


constexpr int kTile = 32;
constexpr float kLazy = 8.0f;  // rescale threshold (log2 units)
constexpr int kCombineThreads = 256;

// Workgroup shape: W waves, each keeping PF tiles of loads in registers
// (32 VGPRs per tile at head_dim 64, 64 at 128).
template <int D>
struct DecodeShape;
template <>
struct DecodeShape<64> {
  static constexpr int W = 4, PF = 1;
};
template <>
struct DecodeShape<128> {
  static constexpr int W = 4, PF = 1;
};
constexpr int kCombineChunk = 16;  // most split partials loaded together by the combine
constexpr int kSplitLocal = 1;     // buffer cache policy sc0: past the CU's L1, from the L2
constexpr int kSplitCtrPitch = 32; // in-kernel split merge: one counter per 128-byte line

// A buffer over one of the split partial arrays: n_units * nhm * per floats
// (under 2 GiB: the launch checks).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t split_rsrc(float* base, const DecodeArgs& a,
                                                             int per) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, a.n_units * a.nhm * per * 4, 0x00020000);
}

template <int D>
struct Tile {
  static constexpr int ND = D / 32;       // 32-wide d blocks of QK
  static constexpr int VCH = D / 8;       // 16-byte chunks per V row
  static constexpr int VROWS = 64 / VCH;  // V rows per wave-wide load
  static constexpr int VLOADS = kTile / VROWS;
  half8_t k[2][ND];
  half8_t v[VLOADS];
};

// q rows of this lane's head and their RoPE table entries, loaded before the
// first K/V tiles so that waiting for them (the vector-memory counter is
// in-order) does not wait for the tiles.  Lane (col, grp) holds
// q[h][32*db + 8*grp + j] for db < D/32, j < 8 (zero for lanes beyond the
// group), the D/8 table entries its pairs need and, with QK-norm, the q norm
// weights of its elements.
template <int D>
struct QRaw {
  float q[D / 32][8];
  float c[D / 8], s[D / 8];
  float w[D / 32][8];
  const float* row;  // this lane's q row
};

// Buffer cache policy sc1: device scope, read past the L2 (data another XCD
// wrote in the same launch).
constexpr int kDevScope = 16;

// A buffer resource over n bytes at p (loads with a cache policy).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* p, size_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)n, 0x00020000);
}

// COH: q, k and v were written by other workgroups of the same launch (the
// fused q/k/v + attention launch): loaded at device scope.
template <int D, bool QKN, bool COH = false>
__device__ __forceinline__ void load_q_raw(const DecodeArgs& a, int li, int kvh, int G, int h0,
                                           int nh, int col, int grp, QRaw<D>& r) {
  constexpr int ND = D / 32;
  const bool valid = col < nh;  // lanes past the group load head h0's row; rope_q zeroes them
  const float* qrow =
      a.q + (size_t)li * a.n_heads * D + (size_t)(kvh * G + h0 + (valid ? col : 0)) * D;
  r.row = qrow;
#pragma unroll
  for (int db = 0; db < ND; ++db) {
    float4 x0, x1;
    if constexpr (COH) {
      // one launch layer: q is [n_heads * D] floats
      const __amdgpu_buffer_rsrc_t rq = raw_rsrc(a.q, (size_t)a.n_heads * D * sizeof(float));
      const int off = (int)((qrow - a.q) + 32 * db + 8 * grp) * 4;
      const float4_t y0 = __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, kDevScope);
      const float4_t y1 = __builtin_amdgcn_raw_buffer_load_b128(rq, off + 16, 0, kDevScope);
      x0 = make_float4(y0[0], y0[1], y0[2], y0[3]);
      x1 = make_float4(y1[0], y1[1], y1[2], y1[3]);
    } else {
      x0 = *(const float4*)(qrow + 32 * db + 8 * grp);
      x1 = *(const float4*)(qrow + 32 * db + 8 * grp + 4);
    }
    r.q[db][0] = x0.x, r.q[db][1] = x0.y, r.q[db][2] = x0.z, r.q[db][3] = x0.w;
    r.q[db][4] = x1.x, r.q[db][5] = x1.y, r.q[db][6] = x1.z, r.q[db][7] = x1.w;
  }
  if (QKN) {
    const float* wq = a.qn + (size_t)li * D;
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      const float4 w0 = *(const float4*)(wq + 32 * db + 8 * grp);
      const float4 w1 = *(const float4*)(wq + 32 * db + 8 * grp + 4);
      r.w[db][0] = w0.x, r.w[db][1] = w0.y, r.w[db][2] = w0.z, r.w[db][3] = w0.w;
      r.w[db][4] = w1.x, r.w[db][5] = w1.y, r.w[db][6] = w1.z, r.w[db][7] = w1.w;
    }
  }
  const float* cr = a.cos_t + (size_t)a.pos * (D / 2);
  const float* sr = a.sin_t + (size_t)a.pos * (D / 2);
  if (a.rope_type == PLH_ROPE_QWEN) {
    // pairs (i, i + D/2), i = 32*db + 8*grp + j for db < ND/2
#pragma unroll
    for (int db = 0; db < ND / 2; ++db)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float4 c4 = *(const float4*)(cr + 32 * db + 8 * grp + 4 * hh);
        float4 s4 = *(const float4*)(sr + 32 * db + 8 * grp + 4 * hh);
        const int o = db * 8 + 4 * hh;
        r.c[o] = c4.x, r.c[o + 1] = c4.y, r.c[o + 2] = c4.z, r.c[o + 3] = c4.w;
        r.s[o] = s4.x, r.s[o + 1] = s4.y, r.s[o + 2] = s4.z, r.s[o + 3] = s4.w;
      }
  } else {
    // pairs (2i, 2i+1), i = 16*db + 4*grp + jj
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      float4 c4 = *(const float4*)(cr + 16 * db + 4 * grp);
      float4 s4 = *(const float4*)(sr + 16 * db + 4 * grp);
      const int o = db * 4;
      r.c[o] = c4.x, r.c[o + 1] = c4.y, r.c[o + 2] = c4.z, r.c[o + 3] = c4.w;
      r.s[o] = s4.x, r.s[o + 1] = s4.y, r.s[o + 2] = s4.z, r.s[o + 3] = s4.w;
    }
  }
}

// Rotates the loaded q rows in place with the reference's pairing (after
// QK-norm when enabled); lanes beyond the group (valid false) get zero rows.
template <int D, bool QKN>
__device__ __forceinline__ void rope_q(int rope_type, bool valid, int grp, float eps,
                                       QRaw<D>& r) {
  constexpr int ND = D / 32;
  if (QKN) {
    const float sc = rms_scale_grp<D>(r.row, grp, eps);
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float t = r.q[db][j] * sc;
        r.q[db][j] = t * r.w[db][j];
      }
  }
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int j = 0; j < 8; ++j) r.q[db][j] = valid ? r.q[db][j] : 0.f;
  if (rope_type == PLH_ROPE_QWEN) {
#pragma unroll
    for (int db = 0; db < ND / 2; ++db)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        rope_rotate(r.q[db][j], r.q[db + ND / 2][j], r.c[db * 8 + j], r.s[db * 8 + j]);
  } else {
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        rope_rotate(r.q[db][2 * jj], r.q[db][2 * jj + 1], r.c[db * 4 + jj], r.s[db * 4 + jj]);
  }
}

// Inputs of the appended row pos that lane `lane` of the owner's wave 0 needs:
// rope pairs i = lane (+64) of k, and v elements lane (+64).
template <int D>
struct RowRaw {
  static constexpr int NP = (D / 2 + 63) / 64;
  static_assert(NP == 1, "one rope pair per lane");
  static constexpr int NV = (D + 63) / 64;
  float k0[NP], k1[NP], c[NP], s[NP];
  float w0[NP], w1[NP];  // k norm weights of the pair (QK-norm)
  float v[NV];
  const float* kin;      // the k row (QK-norm sums)
};

template <int D, bool QKN, bool COH = false>
__device__ __forceinline__ void load_row_raw(const DecodeArgs& a, int li, int kvh, int lane,
                                             RowRaw<D>& r) {
  const int kv_dim = a.n_kv_heads * D;
  const float* kin = a.k + (size_t)li * kv_dim + (size_t)kvh * D;
  const float* vin = a.v + (size_t)li * kv_dim + (size_t)kvh * D;
  const float* cr = a.cos_t + (size_t)a.pos * (D / 2);
  const float* sr = a.sin_t + (size_t)a.pos * (D / 2);
  r.kin = kin;
#pragma unroll
  for (int u = 0; u < RowRaw<D>::NP; ++u) {
    const int i = min(lane + 64 * u, D / 2 - 1);
    const int i0 = (a.rope_type == PLH_ROPE_QWEN) ? i : 2 * i;
    const int i1 = (a.rope_type == PLH_ROPE_QWEN) ? i + D / 2 : 2 * i + 1;
    if constexpr (COH) {
      // one launch layer: k and v are [n_kv_heads * D] floats
      const __amdgpu_buffer_rsrc_t rk = raw_rsrc(a.k, (size_t)kv_dim * sizeof(float));
      r.k0[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          rk, (kvh * D + i0) * 4, 0, kDevScope));
      r.k1[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          rk, (kvh * D + i1) * 4, 0, kDevScope));
    } else {
      r.k0[u] = kin[i0];
      r.k1[u] = kin[i1];
    }
    r.c[u] = cr[i];
    r.s[u] = sr[i];
    if (QKN) {
      r.w0[u] = a.kn[(size_t)li * D + i0];
      r.w1[u] = a.kn[(size_t)li * D + i1];
    }
  }
#pragma unroll
  for (int u = 0; u < RowRaw<D>::NV; ++u) {
    if constexpr (COH) {
      const __amdgpu_buffer_rsrc_t rv = raw_rsrc(a.v, (size_t)kv_dim * sizeof(float));
      r.v[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          rv, (kvh * D + min(lane + 64 * u, D - 1)) * 4, 0, kDevScope));
    } else {
      r.v[u] = vin[min(lane + 64 * u, D - 1)];
    }
  }
}

// QK-norm of the appended k row held as rope pairs by the wave (lane i holds
// pair i); every lane forms the scale from the row in memory.
template <int D>
__device__ __forceinline__ void qk_norm_row(int grp, float eps, RowRaw<D>& r) {
  const float sc = rms_scale_grp<D>(r.kin, grp, eps);
  float t = r.k0[0] * sc;
  r.k0[0] = t * r.w0[0];
  t = r.k1[0] * sc;
  r.k1[0] = t * r.w1[0];
}

// Issues the loads of the 32-row tile starting at t0; rows past tlast are
// clamped to tlast (always a valid cached row) and masked out of the softmax.
template <int D>
__device__ __forceinline__ void load_tile(Tile<D>& T, const uint16_t* kbase,
                                          const uint16_t* vbase, int kv_dim, int t0, int tlast,
                                          int lane, int col, int grp) {
  using TT = Tile<D>;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int row = min(t0 + 16 * rb + col, tlast);
    const uint16_t* p = kbase + (size_t)row * kv_dim + 8 * grp;
#pragma unroll
    for (int db = 0; db < TT::ND; ++db) T.k[rb][db] = *(const half8_t*)(p + 32 * db);
  }
#pragma unroll
  for (int i = 0; i < TT::VLOADS; ++i) {
    const int row = min(t0 + i * TT::VROWS + lane / TT::VCH, tlast);
    T.v[i] = *(const half8_t*)(vbase + (size_t)row * kv_dim + 8 * (lane % TT::VCH));
  }
}

template <int D>
__device__ __forceinline__ void process_tile(const Tile<D>& T, const half8_t (&qhi)[D / 32],
                                             const half8_t (&qlo)[D / 32], _Float16* vt, int t0,
                                             int tlast, int lane, int col, int grp, float sscale,
                                             half8_t ones, float& ms, float4_t& lsum,
                                             float4_t (&o)[D / 16]) {
  using TT = Tile<D>;
  constexpr int NO = D / 16;
  constexpr int VP = D + 16;
  float4_t s[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    s[rb] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < TT::ND; ++db) {
      s[rb] = mfma16x16x32(T.k[rb][db], qhi[db], s[rb]);
      s[rb] = mfma16x16x32(T.k[rb][db], qlo[db], s[rb]);
    }
  }
  // V rows into the wave's LDS tile, row-major
#pragma unroll
  for (int i = 0; i < TT::VLOADS; ++i)
    *(half8_t*)(vt + (i * TT::VROWS + lane / TT::VCH) * VP + 8 * (lane % TT::VCH)) = T.v[i];

  // online softmax over this tile (log2 domain); slot j holds tile row
  // 4*grp + j (j < 4) or 16 + 4*grp + j - 4
  float u[8];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) u[4 * rb + r] = s[rb][r];
  if (t0 + kTile - 1 > tlast) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int t = t0 + (j < 4 ? 4 * grp + j : 12 + 4 * grp + j);
      if (t > tlast) u[j] = -INFINITY;
    }
  }
  float tmax = u[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) tmax = vmax(tmax, u[j]);
  tmax = max_xor32(max_xor16(tmax));
  const float tms = tmax * sscale;
  if (__ballot(tms > ms + kLazy)) {
    const float mnew = fmaxf(ms, tms);
    const float alpha = fast_exp2(ms - mnew);
    ms = mnew;
    lsum *= alpha;
#pragma unroll
    for (int ob = 0; ob < NO; ++ob) o[ob] *= alpha;
  }
  half8_t ph, pl;
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const float p0 = fast_exp2(u[j] * sscale - ms);
    const float p1 = fast_exp2(u[j + 1] * sscale - ms);
    half2_t hi, lo;
    split_pair_rtz(p0, p1, hi, lo);
    ph[j] = hi[0], ph[j + 1] = hi[1];
    pl[j] = lo[0], pl[j + 1] = lo[1];
  }
  lsum = mfma16x16x32(ones, ph, lsum);
  lsum = mfma16x16x32(ones, pl, lsum);

  // transposing reads: rows 4*grp + col/4 and 16 + 4*grp + col/4, chunk col%4
  const _Float16* vr = vt + (4 * grp + (col >> 2)) * VP + 4 * (col & 3);
#pragma unroll
  for (int ob = 0; ob < NO; ++ob) {
    const half4_t v0 = lds_read_tr4(vr + 16 * ob);
    const half4_t v1 = lds_read_tr4(vr + 16 * VP + 16 * ob);
    const half8_t va = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
    o[ob] = mfma16x16x32(va, ph, o[ob]);
    o[ob] = mfma16x16x32(va, pl, o[ob]);
  }
}

// Rotates the lane's q elements (after QK-norm when enabled) and splits them
// into fp16 hi + lo MFMA operands.  The column's range for the split is a
// power-of-two scale (1 unless some |q| >= 2^15), folded into its score
// scale: the return value is that column's 2^e.
template <int D, bool QKN>
__device__ __forceinline__ float split_q(const DecodeArgs& a, bool valid, int grp, QRaw<D>& qr,
                                         half8_t (&qhi)[D / 32], half8_t (&qlo)[D / 32]) {
  constexpr int ND = D / 32;
  rope_q<D, QKN>(a.rope_type, valid, grp, a.norm_eps, qr);
  float amax = 0.f;
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = vmax(amax, fabsf(qr.q[db][j]));
  amax = max_xor32(max_xor16(amax));
  float qup;
  const float qdown = q_range_scale(amax, &qup);
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      _Float16 hi, lo;
      split_hi_lo(qr.q[db][j] * qdown, hi, lo);
      qhi[db][j] = hi;
      qlo[db][j] = lo;
    }
  return qup;
}

// Row pos of the group's kv head (one wave): k rotated with table row pos
// (after QK-norm when enabled), both rows rounded with the reference's
// fp32_to_fp16 and stored to the caches, their fp32 values kept in LDS
// (knew, vnew) and the row's scaled score against every q head of the block
// (fp32 q, rotated) in mnew[col].
template <int D, bool QKN>
__device__ __forceinline__ void append_new_row(const DecodeArgs& a, int li, int kvh, size_t row0,
                                               int lane, int col, int grp, const QRaw<D>& qr,
                                               RowRaw<D>& rr, float* knew, float* vnew,
                                               float* mnew) {
  constexpr int ND = D / 32;
  const int kv_dim = a.n_kv_heads * D;
  if (QKN) qk_norm_row<D>(grp, a.norm_eps, rr);
  uint16_t* krow = a.kc + (row0 + a.pos) * kv_dim + (size_t)kvh * D;
  uint16_t* vrow = a.vc + (row0 + a.pos) * kv_dim + (size_t)kvh * D;
#pragma unroll
  for (int u = 0; u < RowRaw<D>::NP; ++u) {
    const int i = lane + 64 * u;
    if (i < D / 2) {
      const int i0 = (a.rope_type == PLH_ROPE_QWEN) ? i : 2 * i;
      const int i1 = (a.rope_type == PLH_ROPE_QWEN) ? i + D / 2 : 2 * i + 1;
      float k0 = rr.k0[u], k1 = rr.k1[u];
      rope_rotate(k0, k1, rr.c[u], rr.s[u]);
      const uint16_t b0 = f16_bits_rha(k0), b1 = f16_bits_rha(k1);
      krow[i0] = b0;
      krow[i1] = b1;
      if (a.k_rows) {
        uint16_t* kr = a.k_rows + (size_t)li * kv_dim + (size_t)kvh * D;
        kr[i0] = b0;
        kr[i1] = b1;
      }
      knew[i0] = f16_bits_to_f32(b0);
      knew[i1] = f16_bits_to_f32(b1);
    }
  }
#pragma unroll
  for (int u = 0; u < RowRaw<D>::NV; ++u) {
    const int d = lane + 64 * u;
    if (d < D) {
      const uint16_t b = f16_bits_rha(rr.v[u]);
      vrow[d] = b;
      if (a.v_rows) a.v_rows[(size_t)li * kv_dim + (size_t)kvh * D + d] = b;
      vnew[d] = f16_bits_to_f32(b);
    }
  }
  // knew is written and read by this wave only; order the LDS accesses
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  float sc = 0.f;
#pragma unroll
  for (int db = 0; db < ND; ++db)
#pragma unroll
    for (int j = 0; j < 8; ++j) sc = __builtin_fmaf(qr.q[db][j], knew[32 * db + 8 * grp + j], sc);
  sc += shfl_xor_f(sc, 16);
  sc += shfl_xor_f(sc, 32);
  if (grp == 0) mnew[col] = sc * a.score_scale;
}

// The fused q/k/v + attention launch (gemv.hip): group g's attention
// workgroup waits until every GEMV workgroup whose rows of q, k or v belong
// to the group has stored them (device scope) and counted itself in on
// ctr[g * kFuseCtrPitch].  Segment s (q, k, v) has wg_rows matrix rows per
// GEMV workgroup and group_rows rows per group; a workgroup counts once for
// every group its rows meet.  One layer per launch, one head block per kv
// head (group g = kv head g).
constexpr int kFuseCtrPitch = 32;
struct FuseWait {
  unsigned* ctr;
  int wg_rows[3];
  int group_rows[3];
};
// GEMV workgroups of wg_rows rows whose rows meet [a, b)
__device__ __forceinline__ int fuse_span(int a, int b, int wg_rows) {
  return (b - 1) / wg_rows - a / wg_rows + 1;
}

// Thread 0 of an attention workgroup: returns once every producer of group
// g's rows of q, k and v has counted in.  They are all dispatched eventually
// (the launch's attention workgroups come first and take one slot each), so
// the wait ends; the poll count only bounds it outright.  The poll is an
// atomic, read where the counts are kept.
__device__ __forceinline__ void fuse_wait(const FuseWait& fw, int g) {
  const int want = fuse_span(g * fw.group_rows[0], (g + 1) * fw.group_rows[0], fw.wg_rows[0]) +
                   fuse_span(g * fw.group_rows[1], (g + 1) * fw.group_rows[1], fw.wg_rows[1]) +
                   fuse_span(g * fw.group_rows[2], (g + 1) * fw.group_rows[2], fw.wg_rows[2]);
  unsigned* c = fw.ctr + g * kFuseCtrPitch;
  for (int it = 0; it < (1 << 22); ++it) {
    if (__hip_atomic_fetch_add(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >=
        (unsigned)want)
      break;
    __builtin_amdgcn_s_sleep(2);
  }
}
// Zeroes group g's count for the next launch, once no workgroup of this
// launch waits on it any more.
__device__ __forceinline__ void fuse_reset(const FuseWait& fw, int g) {
  __hip_atomic_store(fw.ctr + g * kFuseCtrPitch, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// While the projections run: the cached rows [tb, te) of a group come into
// this XCD's L2 (one 16-byte load per 128-byte line of each K and V row,
// straight into a scratch LDS buffer), so the tiles after the first are read
// from the L2.  Waited for here: the waves only wait next.
template <int D>
__device__ __forceinline__ void fuse_warm_rows(const uint16_t* kbase, const uint16_t* vbase,
                                               int kv_dim, int tb, int te, int nthreads) {
  typedef __attribute__((address_space(3))) void* lds_ptr;
  typedef __attribute__((address_space(1))) void* global_ptr;
  __shared__ __align__(16) unsigned char s_warm[1024];
  constexpr int kLines = D / 64;  // 128-byte lines per fp16 row
  for (int i = threadIdx.x; i < (te - tb) * kLines; i += nthreads) {
    const int t = tb + i / kLines, part = i - (i / kLines) * kLines;
    const size_t off = (size_t)t * kv_dim + 64 * part;
    __builtin_amdgcn_global_load_lds((global_ptr)(kbase + off), (lds_ptr)s_warm, 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_ptr)(vbase + off), (lds_ptr)s_warm, 16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0);
}

// The split kernel's body.  PFR: the launch also carries the prefetch
// workgroups of pl (attn_decode_pf_kernel); launches without them take the
// smaller argument block of attn_decode_kernel.  FUSED: one unsplit group
// per workgroup id of a fused launch, whose q, k and v come from the same
// launch's GEMV workgroups (fw).
template <int D, bool QKN, bool PFR, bool FUSED = false>
__device__ __forceinline__ void attn_decode_body(const DecodeArgs& a, const PfLaunch& pl,
                                                 const FuseWait& fw = FuseWait{}) {
  static_assert(!FUSED || (!QKN && !PFR), "fused launches: no QK-norm, no prefetch role");
  constexpr int kWaves = DecodeShape<D>::W;
  constexpr int kThreads = 64 * kWaves;
  constexpr int ND = D / 32;          // 32-wide d blocks of QK
  constexpr int NO = D / 16;          // 16-wide d blocks of PV
  constexpr int VP = D + 16;          // LDS pitch of a V tile row (halves): the 4 rows
                                      // of a transposing read land in disjoint banks
  constexpr int kVtileHalves = kWaves * kTile * VP;
  constexpr int kCombFloats = kWaves * 16 * (D + 2);
  constexpr int kSmemBytes =
      (kVtileHalves * 2 > kCombFloats * 4) ? kVtileHalves * 2 : kCombFloats * 4;
  __shared__ __align__(16) unsigned char smem[kSmemBytes];
  __shared__ int s_merge;

#define PLH_SPLIT_ARGS(a)                                                                        \
  "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.kc), "s"(a.vc), "s"(a.cos_t), "s"(a.sin_t), "s"(a.out),   \
      "s"(a.part_o), "s"(a.part_m), "s"(a.part_l), "s"(a.layer0), "s"(a.n_heads),               \
      "s"(a.n_kv_heads), "s"(a.max_seq_len), "s"(a.pos), "s"(a.rope_type), "s"(a.n_hblk),       \
      "s"(a.nhm), "s"(a.n_split), "s"(a.split_len), "s"(a.n_units), "s"(a.per_xcd),            \
      "s"(a.score_scale), "s"(a.k_rows), "s"(a.v_rows), "s"(a.qn), "s"(a.kn), "s"(a.norm_eps),  \
      "s"(a.G), "s"(a.fd_split.m), "s"(a.fd_split.sh), "s"(a.fd_hblk.m), "s"(a.fd_hblk.sh),     \
      "s"(a.fd_kvh.m), "s"(a.fd_kvh.sh), "s"(a.split_merge), "s"(a.split_ctr)
  if constexpr (PFR) {
    // the prefetch split from the same batch of argument loads
    PLH_ARGS_NOW(PLH_SPLIT_ARGS(a), "s"(pl.n_main));
    static_assert(kSmemBytes >= kPfLdsBytes, "prefetch workgroups use the kernel's LDS");
    if (l2_prefetch_role(pl.plan, pl.n_main, kWaves, smem)) return;
  } else {
    PLH_ARGS_NOW(PLH_SPLIT_ARGS(a));
  }
#undef PLH_SPLIT_ARGS
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;

  // XCD-aware unit order: consecutive workgroup ids go to different XCDs, so
  // each XCD takes a contiguous range of units (whole groups: per_xcd is a
  // multiple of n_split) and a group's splits share one L2.
  const int unit =
      FUSED ? (int)blockIdx.x : (int)(blockIdx.x & 7) * a.per_xcd + (int)(blockIdx.x >> 3);
  if (unit >= a.n_units) return;
  const int group = (int)fdiv(unit, a.fd_split);
  const int split = unit - group * a.n_split;
  const int gh = (int)fdiv(group, a.fd_hblk);  // group / n_hblk
  const int hblk = group - gh * a.n_hblk;
  const int li = (int)fdiv(gh, a.fd_kvh);
  const int kvh = gh - li * a.n_kv_heads;
  const int layer = a.layer0 + li;
  const int G = a.G;
  const int h0 = hblk * 16;
  const int nh = min(16, G - h0);
  const int kv_dim = a.n_kv_heads * D;
  const int pos = a.pos;
  const bool owner = split == a.n_split - 1;

  // ---- loads: q (and the owner's new-row inputs) first, then the first tiles
  const int tb = split * a.split_len;
  const int te = min(tb + a.split_len, pos);   // cached rows [tb, te); row pos is new
  const int tlast = te - 1;
  const size_t row0 = (size_t)layer * a.max_seq_len;
  const uint16_t* kbase = a.kc + row0 * kv_dim + (size_t)kvh * D;
  const uint16_t* vbase = a.vc + row0 * kv_dim + (size_t)kvh * D;
  constexpr int kStride = kWaves * kTile;
  const int tw = tb + wave * kTile;  // this wave's first row; its tiles are kStride apart
  const bool new_row = owner && wave == 0;

  // Rolling prefetch of depth PF: tile i of the wave lives in buffer i % PF,
  // and refilling a buffer with tile i + PF starts as soon as tile i is done.
  // Every load is issued unconditionally (tiles past the range re-read row
  // tlast, or row 0 when the split has no cached rows, and are masked or
  // skipped), so the compiler's wait counts stay exact: the q rotation waits
  // for q alone (issued first), and the prefetch is never drained early.
  // A fused launch issues its first tiles (cached rows, ready) before it
  // waits for q, k and v (two tiles in flight there measured the same).
  constexpr int PF = DecodeShape<D>::PF;
  const bool has_rows = te > tb;
  const int tclamp = has_rows ? tlast : 0;
  Tile<D> buf[PF];
  QRaw<D> qr;
  RowRaw<D> rr;  // the new row's inputs, used by the owner's wave 0 only
  if constexpr (FUSED) {
#pragma unroll
    for (int j = 0; j < PF; ++j)
      load_tile<D>(buf[j], kbase, vbase, kv_dim, tw + j * kStride, tclamp, lane, col, grp);
    fuse_warm_rows<D>(kbase, vbase, kv_dim, tb, te, kThreads);
    if (tid == 0) {
      fuse_wait(fw, kvh);
      fuse_reset(fw, kvh);  // this group's only waiter
    }
    __syncthreads();
    load_q_raw<D, QKN, true>(a, li, kvh, G, h0, nh, col, grp, qr);
    load_row_raw<D, QKN, true>(a, li, kvh, lane, rr);
  } else {
    load_q_raw<D, QKN>(a, li, kvh, G, h0, nh, col, grp, qr);
    load_row_raw<D, QKN>(a, li, kvh, lane, rr);
#pragma unroll
    for (int j = 0; j < PF; ++j)
      load_tile<D>(buf[j], kbase, vbase, kv_dim, tw + j * kStride, tclamp, lane, col, grp);
  }

  // ---- q operands: rotated, split into fp16 hi + lo ------------------------
  // The owner's wave 0 also appends row pos (k rotated, both rows rounded)
  // and scores it against the fp32 q rows.
  __shared__ float s_knew[D], s_vnew[D], s_mnew[16];
  half8_t qhi[ND], qlo[ND];
  // keep the scheduler from hoisting q's uses (and their waits) above the tiles
  __builtin_amdgcn_sched_barrier(0);
  const float qup = split_q<D, QKN>(a, col < nh, grp, qr, qhi, qlo);
  if (new_row) append_new_row<D, QKN>(a, li, kvh, row0, lane, col, grp, qr, rr, s_knew, s_vnew, s_mnew);

  // ---- stream the split's cached rows, one tile ahead ----------------------
  _Float16* vt = reinterpret_cast<_Float16*>(smem) + wave * (kTile * VP);
  const float sscale = a.score_scale * qup;       // this lane's column
  float m = kNegBig;                              // running max (scaled, log2 units)
  float4_t lsum = float4_t{0.f, 0.f, 0.f, 0.f};  // running sum (all entries equal)
  half8_t ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = (_Float16)1.0f;
  float4_t o[NO];
#pragma unroll
  for (int ob = 0; ob < NO; ++ob) o[ob] = float4_t{0.f, 0.f, 0.f, 0.f};

  if (has_rows) {
    for (int base = tw; base < te; base += PF * kStride) {
#pragma unroll
      for (int j = 0; j < PF; ++j) {
        const int t0 = base + j * kStride;
        if (t0 < te)
          process_tile<D>(buf[j], qhi, qlo, vt, t0, tlast, lane, col, grp, sscale, ones, m, lsum,
                          o);
        load_tile<D>(buf[j], kbase, vbase, kv_dim, t0 + PF * kStride, tclamp, lane, col, grp);
      }
    }
  }
  const float l = lsum[0];

  __syncthreads();  // V tiles are dead; the LDS now holds the combine slots
  float* cm = reinterpret_cast<float*>(smem);          // [kWaves][16]
  float* cl = cm + kWaves * 16;                        // [kWaves][16]
  float* co = cl + kWaves * 16;                        // [kWaves][16][D]
  if (grp == 0) {
    cm[wave * 16 + col] = m;
    cl[wave * 16 + col] = l;
  }
#pragma unroll
  for (int ob = 0; ob < NO; ++ob)
#pragma unroll
    for (int r = 0; r < 4; ++r) co[(wave * 16 + col) * D + 16 * ob + 4 * grp + r] = o[ob][r];

  __syncthreads();

  // ---- merge the waves (and the new row) of this workgroup -------------------
  const int q_dim = a.n_heads * D;
  float* out_base = a.out + (size_t)li * q_dim + (size_t)(kvh * G + h0) * D;
  for (int idx = tid; idx < nh * D; idx += kThreads) {
    const int h = idx / D, d = idx - (idx / D) * D;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, cm[w * 16 + h]);
    if (owner) M = fmaxf(M, s_mnew[h]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float wt = fast_exp2(cm[w * 16 + h] - M);
      L = __builtin_fmaf(cl[w * 16 + h], wt, L);
      O = __builtin_fmaf(co[(w * 16 + h) * D + d], wt, O);
    }
    if (owner) {
      const float wt = fast_exp2(s_mnew[h] - M);
      L += wt;
      O = __builtin_fmaf(s_vnew[d], wt, O);
    }
    if (a.n_split == 1) {
      out_base[(size_t)h * D + d] = O * (1.0f / L);
    } else if (a.split_merge) {
      // sc0 stores: in the L2 (the merging split's) when they complete; the
      // 32-bit buffer builtins move raw bits
      const int u = unit * a.nhm + h;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(O), split_rsrc(a.part_o, a, D),
                                            (u * D + d) * 4, 0, kSplitLocal);
      if (d == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(M), split_rsrc(a.part_m, a, 1),
                                              u * 4, 0, kSplitLocal);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(L), split_rsrc(a.part_l, a, 1),
                                              u * 4, 0, kSplitLocal);
      }
    } else {
      a.part_o[((size_t)unit * a.nhm + h) * D + d] = O;
      if (d == 0) {
        a.part_m[(size_t)unit * a.nhm + h] = M;
        a.part_l[(size_t)unit * a.nhm + h] = L;
      }
    }
  }
  if (a.n_split == 1 || !a.split_merge) return;

  // ---- the group's last split merges (its splits share this XCD's L2) -----
  // The partials' sc0 stores complete in the L2 before the count goes up;
  // the merger reads them with sc0 (past its L1) and resets the count for
  // the next launch.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  unsigned* ctr = a.split_ctr + group * kSplitCtrPitch;
  if (tid == 0)
    s_merge = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (unsigned)(a.n_split - 1);
  __syncthreads();
  if (!s_merge) return;
  if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int u0 = group * a.n_split;
  const __amdgpu_buffer_rsrc_t ro = split_rsrc(a.part_o, a, D);
  const __amdgpu_buffer_rsrc_t rm = split_rsrc(a.part_m, a, 1);
  const __amdgpu_buffer_rsrc_t rl = split_rsrc(a.part_l, a, 1);
  for (int idx = tid; idx < nh * D; idx += kThreads) {
    const int h = idx / D, d = idx - (idx / D) * D;
    float M = kNegBig, L = 0.f, O = 0.f;
    for (int s0 = 0; s0 < a.n_split; s0 += 8) {
      float mi[8], li[8], oi[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int u = (u0 + min(s0 + j, a.n_split - 1)) * a.nhm + h;
        mi[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rm, u * 4, 0, kSplitLocal));
        li[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rl, u * 4, 0, kSplitLocal));
        oi[j] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(ro, (u * D + d) * 4, 0, kSplitLocal));
      }
      float Mc = M;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < a.n_split) Mc = fmaxf(Mc, mi[j]);
      const float r = fast_exp2(M - Mc);
      L *= r;
      O *= r;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (s0 + j < a.n_split) {
          const float w = fast_exp2(mi[j] - Mc);
          L = __builtin_fmaf(li[j], w, L);
          O = __builtin_fmaf(oi[j], w, O);
        }
      }
      M = Mc;
    }
    out_base[(size_t)h * D + d] = O * (1.0f / L);
  }
}


// ---- stream-K decode with the merge inside the kernel --------------------
//
// The groups' cached rows, in 16-row blocks, are flattened group-major and
// cut into sk_W equal ranges, one per workgroup (about one per CU), so every
// CU streams the same number of bytes whatever the shape.  A range covers
// the end of one group and the start of the next at most a few times; for
// each group segment the workgroup's 4 waves take its 32-row tiles in turn
// with two tiles of loads in flight per wave (a paced stream: the memory
// queues stay short, so q and the first tiles arrive early), merge through
// LDS as the split kernel does, and then either write the output (the only
// producer of the group) or store a partial and count themselves in.  The
// last producer of a group to arrive merges its partials and writes the
// output, so one launch does everything.  Partials that cross XCDs, whose L2
// caches are not coherent with each other, are stored and loaded with
// device-scope cache policy (sc1: written through, read past the L2); when
// every producer of a group runs on one XCD (sk_wx > 0 places the ranges so,
// see the launch) they go through that XCD's L2 instead (sc0: past the CU's
// L1 only).  Either way the stores complete before the arrival counter is
// bumped, the counter is an atomic at device scope, and the merging
// workgroup resets it to zero for the next launch.

// The T blocks are cut into W ranges of q or q + 1 blocks (q = T / W,
// r = T % W: the first r ranges take q + 1): range w starts at w*q + min(w,
// r).  All in 32-bit integers (the host checks T fits): 64-bit division
// would cost the prologue about a thousand instructions.
__device__ __forceinline__ int sk_start(int w, int q, int r) { return w * q + min(w, r); }
__device__ __forceinline__ int sk_owner(int t, const DecodeArgs& a) {
  const int big = a.sk_r * (a.sk_q + 1);
  return t < big ? (int)fdiv(t, a.fd_q1) : a.sk_r + (int)fdiv(t - big, a.fd_q);
}

constexpr int kSkAux = 16;   // buffer cache policy: sc1 (device scope)
constexpr int kSkLocal = 1;  // sc0: past the CU's L1, served by the XCD's L2
// Arrival counters sit one 128-byte line apart: the producers of different
// groups arrive at once, and atomics on one line queue behind each other
// (one Llama-3.2 layer, 8 groups of 32 producers: 161 us per token with the
// counters a line apart, 191 us with them 4 bytes apart).
constexpr int kSkCtrPitch = 32;

// The last producer's merge of a group's np partials (slots slot0..): POL is
// the cache policy the producers stored them with.
template <int D, int POL>
__device__ __forceinline__ void sk_merge_partials(const DecodeArgs& a,
                                                  __amdgpu_buffer_rsrc_t prs, int slot0, int np,
                                                  int h, int d, float* dst) {
  constexpr int PS = D + 4;
  float M = kNegBig, L = 0.f;
  float4_t O = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < np; j0 += 8) {
    float4_t ml[8], oj[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int off = ((slot0 + min(j0 + j, np - 1)) * a.nhm + h) * PS;
      ml[j] = __builtin_amdgcn_raw_buffer_load_b128(prs, (off + D) * 4, 0, POL);
      oj[j] = __builtin_amdgcn_raw_buffer_load_b128(prs, (off + d) * 4, 0, POL);
    }
    float Mc = M;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j0 + j < np) Mc = fmaxf(Mc, ml[j][0]);
    const float r = fast_exp2(M - Mc);
    L *= r;
    O *= r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j0 + j < np) {
        const float wt = fast_exp2(ml[j][0] - Mc);
        L = __builtin_fmaf(ml[j][1], wt, L);
#pragma unroll
        for (int c = 0; c < 4; ++c) O[c] = __builtin_fmaf(oj[j][c], wt, O[c]);
      }
    }
    M = Mc;
  }
  const float inv = 1.0f / L;
  *reinterpret_cast<float4_t*>(dst) = O * inv;
}

template <int D>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const DecodeArgs& a) {
  return __builtin_amdgcn_make_buffer_rsrc(a.sk_part, 0, (int)a.sk_part_bytes, 0x00020000);
}

// The stream-K kernel's body; PFR as for attn_decode_body.
template <int D, bool QKN, int kSkPF, bool PFR>
__device__ __forceinline__ void attn_decode_sk_body(const DecodeArgs& a, const PfLaunch& pl) {
  constexpr int kWaves = 4;
  constexpr int kThreads = 64 * kWaves;
  constexpr int ND = D / 32;
  constexpr int NO = D / 16;
  constexpr int VP = D + 16;
  constexpr int PS = D + 4;  // floats per (slot, head) of a partial: o[D], m, l, pad
  constexpr int kVtileHalves = kWaves * kTile * VP;
  constexpr int kCombFloats = kWaves * 16 * (D + 2);
  constexpr int kSmemBytes =
      (kVtileHalves * 2 > kCombFloats * 4) ? kVtileHalves * 2 : kCombFloats * 4;
  __shared__ __align__(16) unsigned char smem[kSmemBytes];
  __shared__ float s_knew[D], s_vnew[D], s_mnew[16];
  __shared__ int s_last;

#define PLH_SK_ARGS(a)                                                                           \
  "s"(a.q), "s"(a.k), "s"(a.v), "s"(a.kc), "s"(a.vc), "s"(a.cos_t), "s"(a.sin_t), "s"(a.out),   \
      "s"(a.layer0), "s"(a.n_heads), "s"(a.n_kv_heads), "s"(a.max_seq_len), "s"(a.pos),        \
      "s"(a.rope_type), "s"(a.n_hblk), "s"(a.nhm), "s"(a.score_scale), "s"(a.sk_q),             \
      "s"(a.sk_r), "s"(a.sk_nbk), "s"(a.sk_maxp), "s"(a.sk_part), "s"(a.sk_part_bytes),         \
      "s"(a.sk_ctr), "s"(a.k_rows), "s"(a.v_rows), "s"(a.qn), "s"(a.kn), "s"(a.norm_eps),       \
      "s"(a.G), "s"(a.fd_hblk.m), "s"(a.fd_hblk.sh), "s"(a.fd_kvh.m), "s"(a.fd_kvh.sh),         \
      "s"(a.fd_nbk.m), "s"(a.fd_nbk.sh), "s"(a.fd_q.m), "s"(a.fd_q.sh), "s"(a.fd_q1.m),         \
      "s"(a.fd_q1.sh), "s"(a.sk_wx), "s"(a.fd_wx.m), "s"(a.fd_wx.sh), "s"(a.sk_k),              \
      "s"(a.sk_kshift)
  if constexpr (PFR) {
    // the prefetch split from the same batch of argument loads
    PLH_ARGS_NOW(PLH_SK_ARGS(a), "s"(pl.n_main));
    static_assert(kSmemBytes >= kPfLdsBytes, "prefetch workgroups use the kernel's LDS");
    if (l2_prefetch_role(pl.plan, pl.n_main, kWaves, smem)) return;
  } else {
    PLH_ARGS_NOW(PLH_SK_ARGS(a));
  }
#undef PLH_SK_ARGS
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  // sk_wx > 0: ranges x*wx .. x*wx + wx - 1 run on XCD x (workgroup ids x,
  // x + 8, ...: the dispatcher deals workgroups to the XCDs in turn), so
  // most groups' producers share one L2
  const int w = a.sk_wx ? (int)(blockIdx.x & 7) * a.sk_wx + (int)(blockIdx.x >> 3)
                        : (int)blockIdx.x;
  int b0, b1;
  if (a.sk_k) {
    // range j of group g: blocks [j * nbk / k, (j + 1) * nbk / k) of the group
    const int g = w >> a.sk_kshift, j = w & (a.sk_k - 1);
    b0 = g * a.sk_nbk + ((j * a.sk_nbk) >> a.sk_kshift);
    b1 = g * a.sk_nbk + (((j + 1) * a.sk_nbk) >> a.sk_kshift);
  } else {
    b0 = sk_start(w, a.sk_q, a.sk_r);
    b1 = sk_start(w + 1, a.sk_q, a.sk_r);
  }
  const int G = a.G;
  const int kv_dim = a.n_kv_heads * D;
  const int pos = a.pos;
  const int q_dim = a.n_heads * D;
  const __amdgpu_buffer_rsrc_t prs = sk_rsrc<D>(a);

  for (int s0 = b0; s0 < b1;) {
    const int group = (int)fdiv(s0, a.fd_nbk);
    const int gb = group * a.sk_nbk;
    const int s1 = min(b1, gb + a.sk_nbk);
    const int gh = (int)fdiv(group, a.fd_hblk);  // group / n_hblk
    const int hblk = group - gh * a.n_hblk;
    const int li = (int)fdiv(gh, a.fd_kvh);
    const int kvh = gh - li * a.n_kv_heads;
    const int layer = a.layer0 + li;
    const int h0 = hblk * 16;
    const int nh = min(16, G - h0);
    const int tb = (s0 - gb) * 16;
    const int te = min((s1 - gb) * 16, pos);  // cached rows [tb, te); row pos is new
    const bool owner = s1 == gb + a.sk_nbk;   // covers the group's last block

    const int tlast = te - 1;
    const size_t row0 = (size_t)layer * a.max_seq_len;
    const uint16_t* kbase = a.kc + row0 * kv_dim + (size_t)kvh * D;
    const uint16_t* vbase = a.vc + row0 * kv_dim + (size_t)kvh * D;
    constexpr int kStride = kWaves * kTile;
    const int tw = tb + wave * kTile;
    const bool new_row = owner && wave == 0;

    QRaw<D> qr;
    load_q_raw<D, QKN>(a, li, kvh, G, h0, nh, col, grp, qr);
    RowRaw<D> rr;
    load_row_raw<D, QKN>(a, li, kvh, lane, rr);

    const bool has_rows = te > tb;
    const int tclamp = has_rows ? tlast : 0;
    Tile<D> buf[kSkPF];
#pragma unroll
    for (int j = 0; j < kSkPF; ++j)
      load_tile<D>(buf[j], kbase, vbase, kv_dim, tw + j * kStride, tclamp, lane, col, grp);

    half8_t qhi[ND], qlo[ND];
    __builtin_amdgcn_sched_barrier(0);
    const float qup = split_q<D, QKN>(a, col < nh, grp, qr, qhi, qlo);
    if (new_row)
      append_new_row<D, QKN>(a, li, kvh, row0, lane, col, grp, qr, rr, s_knew, s_vnew, s_mnew);

    _Float16* vt = reinterpret_cast<_Float16*>(smem) + wave * (kTile * VP);
    const float sscale = a.score_scale * qup;
    float m = kNegBig;
    float4_t lsum = float4_t{0.f, 0.f, 0.f, 0.f};
    half8_t ones;
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = (_Float16)1.0f;
    float4_t o[NO];
#pragma unroll
    for (int ob = 0; ob < NO; ++ob) o[ob] = float4_t{0.f, 0.f, 0.f, 0.f};

    if (has_rows) {
      for (int base = tw; base < te; base += kSkPF * kStride) {
#pragma unroll
        for (int j = 0; j < kSkPF; ++j) {
          const int t0 = base + j * kStride;
          if (t0 < te)
            process_tile<D>(buf[j], qhi, qlo, vt, t0, tlast, lane, col, grp, sscale, ones, m,
                            lsum, o);
          load_tile<D>(buf[j], kbase, vbase, kv_dim, t0 + kSkPF * kStride, tclamp, lane, col,
                       grp);
        }
      }
    }
    const float l = lsum[0];

    __syncthreads();  // V tiles are dead; the LDS now holds the combine slots
    float* cm = reinterpret_cast<float*>(smem);
    float* cl = cm + kWaves * 16;
    float* co = cl + kWaves * 16;
    if (grp == 0) {
      cm[wave * 16 + col] = m;
      cl[wave * 16 + col] = l;
    }
#pragma unroll
    for (int ob = 0; ob < NO; ++ob)
#pragma unroll
      for (int r = 0; r < 4; ++r) co[(wave * 16 + col) * D + 16 * ob + 4 * grp + r] = o[ob][r];
    __syncthreads();

    // producers of this group: the workgroups owning its first and last block
    const int p0 = a.sk_k ? group << a.sk_kshift : sk_owner(gb, a);
    const int np = a.sk_k ? a.sk_k : sk_owner(gb + a.sk_nbk - 1, a) - p0 + 1;
    // all producers on one XCD: partials and the count stay in its L2
    const bool local = a.sk_wx && fdiv(p0, a.fd_wx) == fdiv(p0 + np - 1, a.fd_wx);

    // ---- merge the waves (and the new row); one float4 of d per thread -----
    float* out_base = a.out + (size_t)li * q_dim + (size_t)(kvh * G + h0) * D;
    const int slot0 = group * a.sk_maxp;
    for (int idx = tid; idx < nh * (D / 4); idx += kThreads) {
      const int h = idx / (D / 4), d = 4 * (idx - h * (D / 4));
      float M = kNegBig;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, cm[ww * 16 + h]);
      if (owner) M = fmaxf(M, s_mnew[h]);
      float L = 0.f;
      float4_t O = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const float wt = fast_exp2(cm[ww * 16 + h] - M);
        L = __builtin_fmaf(cl[ww * 16 + h], wt, L);
        const float4_t x = *reinterpret_cast<const float4_t*>(co + (ww * 16 + h) * D + d);
#pragma unroll
        for (int c = 0; c < 4; ++c) O[c] = __builtin_fmaf(x[c], wt, O[c]);
      }
      if (owner) {
        const float wt = fast_exp2(s_mnew[h] - M);
        L += wt;
#pragma unroll
        for (int c = 0; c < 4; ++c) O[c] = __builtin_fmaf(s_vnew[d + c], wt, O[c]);
      }
      if (np == 1) {
        const float inv = 1.0f / L;
        *reinterpret_cast<float4_t*>(out_base + (size_t)h * D + d) = O * inv;
      } else {
        const int off = ((slot0 + (w - p0)) * a.nhm + h) * PS;
        const float4_t ml = float4_t{M, L, 0.f, 0.f};
        if (local) {
          __builtin_amdgcn_raw_buffer_store_b128(O, prs, (off + d) * 4, 0, kSkLocal);
          if (d == 0) __builtin_amdgcn_raw_buffer_store_b128(ml, prs, (off + D) * 4, 0, kSkLocal);
        } else {
          __builtin_amdgcn_raw_buffer_store_b128(O, prs, (off + d) * 4, 0, kSkAux);
          if (d == 0) __builtin_amdgcn_raw_buffer_store_b128(ml, prs, (off + D) * 4, 0, kSkAux);
        }
      }
    }

    if (np > 1) {
      // every partial store has reached memory before the count goes up
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      // the count is a device-scope atomic on either path
      unsigned* ctr = a.sk_ctr + group * kSkCtrPitch;
      if (tid == 0)
        s_last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(np - 1);
      __syncthreads();
      if (s_last) {
        if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int idx = tid; idx < nh * (D / 4); idx += kThreads) {
          const int h = idx / (D / 4), d = 4 * (idx - h * (D / 4));
          float* dst = out_base + (size_t)h * D + d;
          if (local)
            sk_merge_partials<D, kSkLocal>(a, prs, slot0, np, h, d, dst);
          else
            sk_merge_partials<D, kSkAux>(a, prs, slot0, np, h, d, dst);
        }
      }
    }
    s0 = s1;
    __syncthreads();  // the LDS is reused by the next segment
  }
}

}  // namespace
