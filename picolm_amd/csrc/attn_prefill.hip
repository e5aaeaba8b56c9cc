// attn_prefill.hip -- causal prompt prefill for gfx950.
//
// Replaces model.c:1019-1090.  The reference walks the prompt serially: for
// token bi (position start_pos+bi) it rotates q and k, appends f16(k_rot) and
// f16(v) at cache row start_pos+bi, then attends over rows 0..start_pos+bi.
// Because each token's row depends only on its own k/v, that is the same as
// "append all rows, then causal attention", which is what the two kernels
// here do:
//
//   prefill_append_kernel  rotates k (table row = its position), rounds k_rot
//                          and v with the reference's fp16 rounding and writes
//                          rows start_pos .. start_pos+n_tokens-1;
//   prefill_attn_kernel    flash attention over the cache with fp16 MFMA and
//                          an fp32 online softmax.
//
// Attention unit = (layer, kv head, block of bq prompt tokens).  A workgroup
// of 4 waves runs one unit (or a pair, see prefill_attn_kernel); each wave
// owns 32 "columns", a column being one (token, q head) pair of the block, so
// all q heads of the kv head's GQA group share every K/V tile.  K/V tiles of
// 32 rows are staged in LDS (double-buffered, loaded by the whole workgroup)
// and both products run on v_mfma_f32_32x32x16_f16:
//   S^T[t][c] = K[t][:] . q_c           A = K rows (ds_read_b128), B = q_c hi/lo
//   O^T[d][c] += V^T[d][t] P^T[t][c]    A = V^T (two ds_read_b64_tr_b16), B = P hi/lo
// K rows are stored in LDS with bits 2 and 3 of the row index swapped, which
// leaves each lane holding the softmax weights of exactly the keys its PV
// operand needs, so P never leaves registers.  q and P are split into fp16
// hi + lo parts (two MFMAs each), keeping the products at ~fp32 precision
// (one fp16 rounding of either would cost ~2e-4 and, for q, grow with the
// scores' magnitude).
//
// Softmax bookkeeping per tile is kept short: the 1/sqrt(D)*log2(e) scale is
// folded into q, the QK accumulators start at minus the running maximum (so
// the MFMA yields score - max), the causal mask is applied only on tiles that
// cross a column's last row, and the running maximum is raised (and O, l
// rescaled) only when a new score exceeds it by more than kLazy, so weights
// stay at most 2^kLazy.  Row sums add the weights as rounded for the MFMA
// (hi + lo) with v_dot2_f32_f16 in fp32.
#include <limits.h>
#include <math.h>

#include "attn_common.h"
#include "picolm_hip.h"
#include "plh_internal.h"

using namespace plh;

namespace {

constexpr int kPW = 4;               // waves per attention workgroup
constexpr int kPThreads = 64 * kPW;
constexpr int kPCols = 32 * kPW;     // (token, q head) columns per workgroup
constexpr int kKT = 32;              // K/V rows per tile
constexpr float kLazy = 8.0f;        // rescale threshold (log2 units)

// One thread per (layer, token, kv head, 4 rope pairs): 16-byte loads of k
// and v, and 8-byte fp16 stores.  LLAMA pairs (2i, 2i+1) for i = 4g..4g+3
// cover elements 8g..8g+7; QWEN pairs (i, i + D/2) cover 4g..4g+3 and
// D/2 + 4g..D/2 + 4g+3.
template <int D, bool QKN>
__global__ __launch_bounds__(256) void prefill_append_kernel(PrefillArgs a) {
  constexpr int NG = D / 8;  // groups of 4 pairs per head
  const int kv_dim = a.n_kv_heads * D;
  const long total = (long)a.n_launch_layers * a.n_tokens * a.n_kv_heads * NG;
  const bool qwen = a.rope_type == PLH_ROPE_QWEN;
  // QK-norm: squares of each k row, for the row's own lanes (pitch D + 8
  // keeps the four or eight rows of a wave in disjoint banks)
  constexpr int kSqPitch = D + 8;
  __shared__ __align__(16) float ksq[QKN ? (256 / NG) * kSqPitch : 1];
  for (long idx = (long)blockIdx.x * 256 + threadIdx.x; idx < total;
       idx += (long)gridDim.x * 256) {
    // item idx = ((layer * n_tokens + token) * n_kv_heads + kv head) * NG + g;
    // below 2^31 items the divisions are multiplies (a 64-bit division by a
    // runtime value costs hundreds of instructions)
    const int g = (int)(idx % NG);
    int kvh, tok, li;
    long lt;
    if (a.app32) {
      const uint32_t rest = (uint32_t)idx / NG;
      const uint32_t lt32 = fdiv(rest, a.fd_app_kvh);
      const uint32_t li32 = fdiv(lt32, a.fd_app_tok);
      kvh = (int)(rest - lt32 * (uint32_t)a.n_kv_heads);
      tok = (int)(lt32 - li32 * (uint32_t)a.n_tokens);
      li = (int)li32;
      lt = lt32;
    } else {
      const long rest = idx / NG;
      kvh = (int)(rest % a.n_kv_heads);
      lt = rest / a.n_kv_heads;
      tok = (int)(lt % a.n_tokens);
      li = (int)(lt / a.n_tokens);
    }
    const int pos = a.start_pos + tok;
    const float* kin = a.k + (size_t)lt * kv_dim + (size_t)kvh * D;
    const float* vin = a.v + (size_t)lt * kv_dim + (size_t)kvh * D;
    const size_t out_row =
        ((size_t)(a.layer0 + li) * a.max_seq_len + pos) * kv_dim + (size_t)kvh * D;
    const float4 c4 = *(const float4*)(a.cos_t + (size_t)pos * (D / 2) + 4 * g);
    const float4 s4 = *(const float4*)(a.sin_t + (size_t)pos * (D / 2) + 4 * g);
    const float cc[4] = {c4.x, c4.y, c4.z, c4.w}, ss[4] = {s4.x, s4.y, s4.z, s4.w};
    // element offsets of the two 4-wide pieces this thread owns
    const int e0 = qwen ? 4 * g : 8 * g;
    const int e1 = qwen ? D / 2 + 4 * g : 8 * g + 4;
    const float4 ka = *(const float4*)(kin + e0), kb = *(const float4*)(kin + e1);
    const float4 va = *(const float4*)(vin + e0), vb = *(const float4*)(vin + e1);
    float k8[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
    const float v8[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
    if (QKN) {
      // QK-norm of the k head row before the rotation.  The row's NG lanes
      // (consecutive, one wave) leave their squares in LDS; lane g then forms
      // the running sums of classes 2(g&3) and 2(g&3)+1 in element order and
      // the fold adds those of lanes g^2 and g^1.  LDS operations of a wave
      // complete in order; the waits and clobbers keep the compiler's order.
      float* sq = ksq + (threadIdx.x / NG) * kSqPitch;
      *(float4*)(sq + e0) = make_float4(ka.x * ka.x, ka.y * ka.y, ka.z * ka.z, ka.w * ka.w);
      *(float4*)(sq + e1) = make_float4(kb.x * kb.x, kb.y * kb.y, kb.z * kb.z, kb.w * kb.w);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      const int p = g & 3;
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int m = 0; m < D / 8; ++m) {
        const float2 t = *(const float2*)(sq + 8 * m + 2 * p);
        s0 = s0 + t.x;
        s1 = s1 + t.y;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      const float sc = rms_scale_pairs(
          s0, s1, D, a.norm_eps, [](float v) { return v + __shfl_xor(v, 2, 64); },
          [](float v) { return v + __shfl_xor(v, 1, 64); });
      const float* wk = a.kn + (size_t)li * D;
      const float4 wa = *(const float4*)(wk + e0), wb = *(const float4*)(wk + e1);
      const float w8[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float t = k8[j] * sc;
        k8[j] = t * w8[j];
      }
    }
    if (qwen) {
#pragma unroll
      for (int j = 0; j < 4; ++j) rope_rotate(k8[j], k8[4 + j], cc[j], ss[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) rope_rotate(k8[2 * j], k8[2 * j + 1], cc[j], ss[j]);
    }
    uint16_t kh[8], vh[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      kh[j] = f16_bits_rha(k8[j]);
      vh[j] = f16_bits_rha(v8[j]);
    }
    auto pack = [](const uint16_t* h) {
      uint2 r;
      r.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
      r.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
      return r;
    };
    if (qwen) {
      *(uint2*)(a.kc + out_row + e0) = pack(kh);
      *(uint2*)(a.kc + out_row + e1) = pack(kh + 4);
      *(uint2*)(a.vc + out_row + e0) = pack(vh);
      *(uint2*)(a.vc + out_row + e1) = pack(vh + 4);
    } else {  // e1 = e0 + 4: one 16-byte store each
      const uint2 k0 = pack(kh), k1 = pack(kh + 4), v0 = pack(vh), v1 = pack(vh + 4);
      *(uint4*)(a.kc + out_row + e0) = make_uint4(k0.x, k0.y, k1.x, k1.y);
      *(uint4*)(a.vc + out_row + e0) = make_uint4(v0.x, v0.y, v1.x, v1.y);
    }
  }
}

template <int D>
struct PrefillLds {
  static constexpr int KP = D + 8;          // LDS pitch of a K row (halves): KP/8 is odd,
                                            // so the 8 consecutive rows a ds_read_b128
                                            // serves at once start in distinct 16-byte
                                            // bank groups
  static constexpr int VP = D + 16;         // LDS pitch of a V row: the 4 rows of a
                                            // transposing read land in disjoint 32-byte
                                            // bank groups
  static constexpr int KBUF = kKT * KP;     // one K tile buffer (halves)
  static constexpr int VBUF = kKT * VP;     // one V tile buffer (halves)
  static constexpr int VOFF = 2 * KBUF;     // V buffers follow the two K buffers
  static constexpr int HALVES = 2 * KBUF + 2 * VBUF;
  static constexpr int QSTAGE = kPCols * (D + 4) * 2;  // the staged q block (halves)
};

// Tiles of the q block qb of a launch: its last token's causal limit, in
// 32-row tiles.
__host__ __device__ inline int prefill_unit_tiles(const PrefillArgs& a, int qb) {
  const int last = (qb + 1) * a.bq < a.n_tokens ? (qb + 1) * a.bq : a.n_tokens;
  return (a.start_pos + last + kKT - 1) / kKT;
}

// One unit: the q block qb (tokens qb*bq ..) of one (layer, kv head) group,
// over its K/V tiles [tb, min(te, its tile count)).  slot < 0: the whole
// range, normalised output written to a.out; else one chunk of a split unit,
// whose unnormalised O, running maximum and sum go to partial slot `slot`
// (prefill_merge_kernel combines the chunks).
//
// KS > 1 (prefill_attn_ksplit_kernel, whole units only): the workgroup is KS
// groups of 4 waves, group g taking tiles tb+g, tb+g+KS, ... with its own LDS
// tile buffers; every group runs the same number of iterations (a group past
// the unit's last tile only joins the barrier), and at the end groups 1.. pass
// their (O, running maximum, sum) through LDS to group 0, which merges them
// like prefill_merge_kernel and writes the output.
template <int D, bool QKN, int KS = 1>
__device__ __forceinline__ void prefill_attn_unit(const PrefillArgs& a, _Float16* smem_wg,
                                                  int group, int qb, int tb, int te, int slot) {
  constexpr int NS = D / 16;        // 16-deep k-steps of QK
  constexpr int NDB = D / 32;       // 32-row d blocks of O^T
  constexpr int KP = PrefillLds<D>::KP, VP = PrefillLds<D>::VP;
  constexpr int KBUF = PrefillLds<D>::KBUF, VBUF = PrefillLds<D>::VBUF;
  constexpr int VOFF = PrefillLds<D>::VOFF;
  constexpr int KCH = kKT * D / 8;  // 16-byte chunks of a K (or V) tile
  constexpr int LPT = 2 * KCH / kPThreads;  // chunks per thread: the first LPT/2 are K
  static_assert(KCH % kPThreads == 0, "tile chunks must split evenly over the workgroup");

  // K-split workgroups stage the unit's q block in LDS (their wave groups
  // share it); one-group workgroups load their columns directly, which keeps
  // their register peak (and occupancy) where it was
  constexpr bool kStageQ = KS > 1;
  const int tid = (int)threadIdx.x & (kPThreads - 1);    // thread within its wave group
  const int kg = KS > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x / kPThreads) : 0;
  _Float16* const smem = smem_wg + kg * PrefillLds<D>::HALVES;  // the group's tile buffers
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int kvh = group % a.n_kv_heads;
  const int li = group / a.n_kv_heads;
  const int layer = a.layer0 + li;
  const int G = a.n_heads / a.n_kv_heads;
  const int kv_dim = a.n_kv_heads * D;
  const int q_dim = a.n_heads * D;
  const int i0 = qb * a.bq;
  const int last_tok = min(i0 + a.bq, a.n_tokens) - 1;
  const int n_rows = a.start_pos + last_tok + 1;          // rows [0, n_rows) are needed
  const int n_tiles = min((n_rows + kKT - 1) / kKT, te);

  // this lane's column: token i0+tok, q head kvh*G+hh
  const int c = wave * 32 + col;
  const int tok = c / G, hh = c - (c / G) * G;
  const bool cvalid = tok < a.bq && i0 + tok < a.n_tokens;
  const int tok_c = cvalid ? i0 + tok : last_tok;          // clamped for addressing
  const int p_col = a.start_pos + tok_c;                  // causal limit of the column
  // smallest and largest causal limits among the wave's columns (wave-uniform)
  const int p_min = __builtin_amdgcn_readfirstlane(
      a.start_pos + min(i0 + (wave * 32) / G, last_tok));
  const int p_max = __builtin_amdgcn_readfirstlane(
      a.start_pos + min(i0 + (wave * 32 + 31) / G, last_tok));

  // ---- cooperative tile loads (issued early; stored to LDS after compute) --
  // Chunk u of a thread is tile chunk tid + u*kPThreads: row r, 16-byte piece
  // q8.  K row r goes to LDS row perm(r) (bits 2 and 3 of r swapped), so that
  // lane m of the QK product reads LDS row m and the MFMA's output rows come
  // out in the order the PV product takes its k operands (see below); V rows
  // stay in key order.
  const size_t row0 = (size_t)layer * a.max_seq_len;
  const uint16_t* kbase = a.kc + row0 * kv_dim + (size_t)kvh * D;
  const uint16_t* vbase = a.vc + row0 * kv_dim + (size_t)kvh * D;
  half8_t ld[LPT];
  auto issue_loads = [&](int t0) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int cc = (tid + u * kPThreads) % KCH;
      const int r = cc / (D / 8), q8 = cc % (D / 8);
      const int row = min(t0 + r, n_rows - 1);
      const uint16_t* src = (u < LPT / 2 ? kbase : vbase) + (size_t)row * kv_dim + 8 * q8;
      ld[u] = *(const half8_t*)src;
    }
  };
  int st_off[LPT];
#pragma unroll
  for (int u = 0; u < LPT; ++u) {
    const int cc = (tid + u * kPThreads) % KCH;
    const int r = cc / (D / 8), q8 = cc % (D / 8);
    const int pr = (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
    st_off[u] = u < LPT / 2 ? pr * KP + 8 * q8 : VOFF + r * VP + 8 * q8;
  }
  auto store_lds = [&](int b) {
#pragma unroll
    for (int u = 0; u < LPT; ++u)
      *(half8_t*)&smem[st_off[u] + b * (u < LPT / 2 ? KBUF : VBUF)] = ld[u];
  };
  issue_loads((tb + kg) * kKT);

  // ---- the unit's q block, staged in LDS by coalesced loads.  Token t of
  // the block holds the G heads of this kv head side by side (G*D floats), so
  // column c = t*G + hh is element run c*D.. of the token-major block; it
  // goes to LDS row c (pitch QSP).  Every wave group of a K-split workgroup
  // reads the same staged block.  The staging overlays the tile buffers,
  // which are first written after the barrier that follows all reads.
  constexpr int QSP = D + 4;  // floats per staged column: rows start in distinct banks
  float* const qs = reinterpret_cast<float*>(smem_wg);
  if constexpr (kStageQ) {
    constexpr int kChunks = kPCols * D / 4;  // float4s of a full block
    constexpr int kPer = (kChunks + kPThreads * KS - 1) / (kPThreads * KS);
    const int gch = G * D / 4;                // float4s per token
    const int n_chunks = a.bq * gch;
    const float* qblk = a.q + (size_t)li * a.n_tokens * q_dim + (size_t)kvh * G * D;
    // chunks past the block repeat its last one (the same load and store),
    // so every thread runs the same straight-line code; tokens past the
    // prompt re-read the last token
    float4 qv[kPer];
    uint32_t dst[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int j = min((int)threadIdx.x + u * kPThreads * KS, n_chunks - 1);
      const int t = j / gch, e = 4 * (j - t * gch);  // element of the token's run
      qv[u] = *(const float4*)(qblk + (uint32_t)min(i0 + t, last_tok) * (uint32_t)q_dim + e);
      dst[u] = (uint32_t)((t * G + e / D) * QSP + e % D);
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) *(float4*)(qs + dst[u]) = qv[u];
    __syncthreads();
  }

  // ---- q operand of this lane's column: element 16*s + 8*half + e of the
  // rotated head row, split into fp16 hi + lo, in qh[s][e] and ql[s][e].
  // Columns past the prompt (cvalid false) read a valid row (column 0 of the
  // staged block, or head 0 of the last token) and are never stored; each
  // column's softmax is independent, so they need no mask.
  half8_t qh[NS], ql[NS];
  float qup, qdown;  // 2^e and 2^-e of the column's range scale
  {
    const float* qcol =
        kStageQ ? qs + (cvalid ? c : 0) * QSP + 8 * half
                : a.q + ((size_t)li * a.n_tokens + tok_c) * q_dim +
                      (size_t)(kvh * G + (cvalid ? hh : 0)) * D + 8 * half;
    const float* cr = a.cos_t + (size_t)p_col * (D / 2);
    const float* sr = a.sin_t + (size_t)p_col * (D / 2);
    float qf[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float4 x0 = *(const float4*)(qcol + 16 * s);
      const float4 x1 = *(const float4*)(qcol + 16 * s + 4);
      qf[s][0] = x0.x, qf[s][1] = x0.y, qf[s][2] = x0.z, qf[s][3] = x0.w;
      qf[s][4] = x1.x, qf[s][5] = x1.y, qf[s][6] = x1.z, qf[s][7] = x1.w;
    }
    if (QKN) {
      // QK-norm of the column's q head row before the rotation
      const float* wq = a.qn + (size_t)li * D;
      float w[NS][8];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float4 w0 = *(const float4*)(wq + 16 * s + 8 * half);
        const float4 w1 = *(const float4*)(wq + 16 * s + 8 * half + 4);
        w[s][0] = w0.x, w[s][1] = w0.y, w[s][2] = w0.z, w[s][3] = w0.w;
        w[s][4] = w1.x, w[s][5] = w1.y, w[s][6] = w1.z, w[s][7] = w1.w;
      }
      const float sc = rms_scale_halves<D>(qf, a.norm_eps);
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float t = qf[s][j] * sc;
          qf[s][j] = t * w[s][j];
        }
    }
    if (a.rope_type == PLH_ROPE_QWEN) {
      // pairs (i, i + D/2): elements of k-steps s and s + NS/2
#pragma unroll
      for (int s = 0; s < NS / 2; ++s) {
        const float4 c0 = *(const float4*)(cr + 16 * s + 8 * half);
        const float4 c1 = *(const float4*)(cr + 16 * s + 8 * half + 4);
        const float4 s0 = *(const float4*)(sr + 16 * s + 8 * half);
        const float4 s1 = *(const float4*)(sr + 16 * s + 8 * half + 4);
        const float cc[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const float ss[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) rope_rotate_fused(qf[s][j], qf[s + NS / 2][j], cc[j], ss[j]);
      }
    } else {
      // pairs (2i, 2i+1), i = 8*s + 4*half + j/2
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float4 c4 = *(const float4*)(cr + 8 * s + 4 * half);
        const float4 s4 = *(const float4*)(sr + 8 * s + 4 * half);
        rope_rotate_fused(qf[s][0], qf[s][1], c4.x, s4.x);
        rope_rotate_fused(qf[s][2], qf[s][3], c4.y, s4.y);
        rope_rotate_fused(qf[s][4], qf[s][5], c4.z, s4.z);
        rope_rotate_fused(qf[s][6], qf[s][7], c4.w, s4.w);
      }
    }
    // the softmax scale log2(e)/sqrt(D) goes into q, so that the MFMA
    // produces scores in log2 units, and the column's range for fp16 (a
    // power-of-two scale 2^-e, undone on the scores: 1 unless some |q| *
    // scale >= 2^15), as one factor: scale * 2^-e is exact, and so is x *
    // (scale * 2^-e) = (x * scale) * 2^-e wherever fp16 can hold the result.
    // The column's largest |q * scale| is (largest |q|) * scale (rounding is
    // monotonic); the maximum is a tree of independent steps, not one chain.
    float am[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float x0 = vmax(vmax(fabsf(qf[s][0]), fabsf(qf[s][1])), fabsf(qf[s][2]));
      const float x1 = vmax(vmax(fabsf(qf[s][3]), fabsf(qf[s][4])), fabsf(qf[s][5]));
      am[s] = vmax(vmax(x0, x1), vmax(fabsf(qf[s][6]), fabsf(qf[s][7])));
    }
#pragma unroll
    for (int w = 1; w < NS; w *= 2)
#pragma unroll
      for (int s = 0; s + w < NS; s += 2 * w) am[s] = vmax(am[s], am[s + w]);
    const float amax = max_xor32(am[0]) * a.score_scale;
    qdown = q_range_scale(amax, &qup);
    const float qmul = a.score_scale * qdown;
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        half2_t hi, lo;
        split_pair_rtz(qf[s][j] * qmul, qf[s][j + 1] * qmul, hi, lo);
        qh[s][j] = hi[0], qh[s][j + 1] = hi[1];
        ql[s][j] = lo[0], ql[s][j + 1] = lo[1];
      }
  }

  if (kStageQ) __syncthreads();  // every lane has read its q column: the tile buffers are free
  store_lds(0);
  __syncthreads();

  // Running maximum ms (log2 units) and the accumulators.  Each QK MFMA chain
  // starts from -ms (times the column's 2^-e), so it yields score - ms
  // directly; the maximum test and the exp2 then read the same values, which
  // keeps every weight bounded (<= 2^kLazy) whatever the scores' magnitude.
  // A column is "fresh" until a tile holds one of its unmasked keys; that
  // tile sets ms to its maximum (a whole unit's first tile does, for every
  // column: row 0 is never masked; a later chunk's first tiles may be masked
  // for some columns).
  //
  // Layouts (v_mfma_f32_32x32x16_f16, lane = 32*half + col):
  //   S^T - ms  [32 keys x 32 columns] = K . q^T: A = K rows (LDS row col,
  //             d 16*s + 8*half ..), B = qh[s]; the lane gets column col and
  //             output rows 8*(v/4) + 4*half + v%4, v = 0..15, which through
  //             the K row permutation are keys 16*(v/8) + 8*half + v%8;
  //   O^T [32 d x 32 columns] += V^T . P^T, per d block and per 16 keys j:
  //             A = V^T (d = col, keys 16*j + 8*half + 0..7, two transposing
  //             LDS reads), B = the lane's own weights v = 8*j .. 8*j+7.
  // So P never leaves registers.  Row sums: each lane adds its 16 weights
  // (as rounded for the MFMA) with v_dot2_f32_f16 in fp32; the two halves of
  // a column are added at the end.
  float ms = 0.f;
  // Raise threshold of ms: -inf while the column is fresh (no unmasked key
  // seen yet; ms, the sums and o all 0), kLazy after (one compare per tile)
  float thr = -INFINITY;
  f32x16_t negm = {};               // -ms * 2^-e, the QK accumulator start
  float ls[4] = {0.f, 0.f, 0.f, 0.f};  // this lane's half of the running sum, in 4
                                       // partial sums (independent add chains)
  const bool scaled_cols = __ballot(qup != 1.f) != 0;  // wave-uniform: rare
  f32x16_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x16_t{};
  const int kofs = col * KP + 8 * half;
  // transposing-read address: 16-lane group g reads keys 8*half + (lane%16)/4
  // (+4 for the second read), d 16*(g%2) + 4*(lane%4) .. of the d block
  const int vofs = (8 * half + ((lane & 15) >> 2)) * VP + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const half2_t one2 = {(_Float16)1.0f, (_Float16)1.0f};

  // one tile in buffer b (a constant at each call site, so the LDS offsets
  // fold into the instructions)
  auto tile = [&](const int b, const int it) {   // it: the group's tile, maybe past the end
    const int t0 = it * kKT;
    const bool more = it + KS < n_tiles;
    if (more) issue_loads(t0 + KS * kKT);
    if (it < n_tiles && t0 <= p_max) {  // else every column of the wave is masked here
      f32x16_t s = negm;
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const half8_t kk = *(const half8_t*)&smem[b * KBUF + kofs + 16 * st];
        s = mfma32x32x16(kk, qh[st], s);
        s = mfma32x32x16(kk, ql[st], s);
      }
      float t[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) t[v] = s[v];
      if (scaled_cols) {
#pragma unroll
        for (int v = 0; v < 16; ++v) t[v] *= qup;  // exact: a power of two
      }
      if (t0 + kKT - 1 > p_min) {
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (t0 + 16 * (v / 8) + 8 * half + v % 8 > p_col) t[v] = -INFINITY;
      }
      // the tile maximum as a tree (depth 3, not a chain of 8)
      const float m0 = vmax(vmax(t[0], t[1]), t[2]), m1 = vmax(vmax(t[3], t[4]), t[5]);
      const float m2 = vmax(vmax(t[6], t[7]), t[8]), m3 = vmax(vmax(t[9], t[10]), t[11]);
      const float m4 = vmax(vmax(t[12], t[13]), t[14]);
      const float tmax =
          max_xor32(vmax(vmax(vmax(m0, m1), m2), vmax(vmax(m3, m4), t[15])));
      // fresh columns with an unmasked key take its maximum as ms (nothing
      // accumulated yet); others raise ms by the excess beyond kLazy
      const bool upd = tmax > thr;
      if (__ballot(upd)) {
        const float d = upd ? tmax : 0.f;
        const bool fresh = thr == -INFINITY;
        const float alpha = fresh ? 1.f : fast_exp2(-d);
#pragma unroll
        for (int k = 0; k < 4; ++k) ls[k] *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db] *= alpha;
        thr = upd ? kLazy : thr;
        ms += d;
        const float nm = -ms * qdown;
#pragma unroll
        for (int v = 0; v < 16; ++v) negm[v] = nm;
#pragma unroll
        for (int v = 0; v < 16; ++v) t[v] -= d;
      }
      half8_t ph[2], pl[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          half2_t hi, lo;
          split_pair_rtz(fast_exp2(t[8 * j + e]), fast_exp2(t[8 * j + e + 1]), hi, lo);
          ph[j][e] = hi[0], ph[j][e + 1] = hi[1];
          pl[j][e] = lo[0], pl[j][e + 1] = lo[1];
          ls[2 * j] = __builtin_amdgcn_fdot2(hi, one2, ls[2 * j], false);
          ls[2 * j + 1] = __builtin_amdgcn_fdot2(lo, one2, ls[2 * j + 1], false);
        }
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const _Float16* vp = &smem[VOFF + b * VBUF + vofs + 16 * j * VP + 32 * db];
          const half4_t v0 = lds_read_tr4(vp);
          const half4_t v1 = lds_read_tr4(vp + 4 * VP);
          const half8_t va = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
          o[db] = mfma32x32x16(va, ph[j], o[db]);
          o[db] = mfma32x32x16(va, pl[j], o[db]);
        }
    }
    if (more) store_lds(b ^ 1);
    __syncthreads();
  };
  const int n_iter = (n_tiles - tb + KS - 1) / KS;  // the same for every group
  for (int i = 0; i < n_iter; i += 2) {
    tile(0, tb + i * KS + kg);
    if (i + 1 < n_iter) tile(1, tb + (i + 1) * KS + kg);
  }

  // ---- normalise and write: lane holds d = 32*db + 8*(v/4) + 4*half + v%4 --
  float lsum = add_xor32((ls[0] + ls[1]) + (ls[2] + ls[3]));
  if (KS > 1) {
    // groups 1.. hand (O, m, l) of each column to group 0 through LDS (the
    // tile buffers are dead: the last barrier followed every tile read)
    constexpr int MP = D + 4;  // floats per column
    float* mb = reinterpret_cast<float*>(smem_wg);
    if (kg > 0) {
      float* dst = mb + ((size_t)(kg - 1) * kPCols + c) * MP;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *(float4*)(dst + 32 * db + 8 * r4 + 4 * half) =
              make_float4(o[db][4 * r4], o[db][4 * r4 + 1], o[db][4 * r4 + 2], o[db][4 * r4 + 3]);
      if (half == 0) {
        dst[D] = thr == -INFINITY ? -INFINITY : ms;
        dst[D + 1] = lsum;
      }
    }
    __syncthreads();
    if (kg > 0) return;
    // group 0 always holds the unit's first tile (row 0, never masked), so
    // its maximum is finite
    float M = ms;
#pragma unroll
    for (int g = 1; g < KS; ++g) M = vmax(M, mb[((size_t)(g - 1) * kPCols + c) * MP + D]);
    const float w0 = fast_exp2(ms - M);
    lsum *= w0;
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] *= w0;
#pragma unroll
    for (int g = 1; g < KS; ++g) {
      const float* src = mb + ((size_t)(g - 1) * kPCols + c) * MP;
      const float wg = fast_exp2(src[D] - M);  // 0 for a group that saw no key
      lsum = __builtin_fmaf(src[D + 1], wg, lsum);
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const float4 x = *(const float4*)(src + 32 * db + 8 * r4 + 4 * half);
          o[db][4 * r4 + 0] = __builtin_fmaf(x.x, wg, o[db][4 * r4 + 0]);
          o[db][4 * r4 + 1] = __builtin_fmaf(x.y, wg, o[db][4 * r4 + 1]);
          o[db][4 * r4 + 2] = __builtin_fmaf(x.z, wg, o[db][4 * r4 + 2]);
          o[db][4 * r4 + 3] = __builtin_fmaf(x.w, wg, o[db][4 * r4 + 3]);
        }
    }
  }
  if (slot >= 0) {
    // a chunk's partial: O, ms (-inf for a column with no unmasked key in the
    // chunk) and the sum, per column of the unit
    if (cvalid) {
      const size_t pc = (size_t)slot * kPCols + c;
      float* po = a.part_o + pc * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *(float4*)(po + 32 * db + 8 * r4 + 4 * half) =
              make_float4(o[db][4 * r4], o[db][4 * r4 + 1], o[db][4 * r4 + 2], o[db][4 * r4 + 3]);
      if (half == 0) {
        a.part_m[pc] = thr == -INFINITY ? -INFINITY : ms;
        a.part_l[pc] = lsum;
      }
    }
    return;
  }
  if (cvalid) {
    const float inv = __builtin_amdgcn_rcpf(lsum);  // v_rcp_f32: within 1 ulp
    float* orow = a.out + ((size_t)li * a.n_tokens + i0 + tok) * a.out_stride +
                  (size_t)(kvh * G + hh) * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        float4_t w;
        w[0] = o[db][4 * r4 + 0] * inv;
        w[1] = o[db][4 * r4 + 1] * inv;
        w[2] = o[db][4 * r4 + 2] * inv;
        w[3] = o[db][4 * r4 + 3] * inv;
        float4_t* dst = (float4_t*)(orow + 32 * db + 8 * r4 + 4 * half);
        // K-split workgroups run one-layer launches: streaming stores there
        // leave less in L2 for the end-of-launch write-back (per-layer
        // TinyLlama 433 -> 420 us); the many-workgroup launches lose with them
        if constexpr (KS > 1)
          __builtin_nontemporal_store(w, dst);
        else
          *dst = w;
      }
  }
}

// Workgroup = one q block, or (a.paired) a pair of q blocks of one (layer, kv
// head) group: the heavy block nq-1-p, then its mirror p, whose K/V tiles are
// a prefix of the heavy block's and still in L2; pairs give every workgroup
// about the same number of tiles.  Single blocks run heaviest first
// (longest-first keeps the end of the launch even when there are several
// workgroups per slot), or (a.split_tiles) as chunks of split_tiles tiles.
// XCD-aware order with 32 groups or more: each XCD takes whole groups (block
// b runs on XCD b % 8), so a group's K/V tiles stay in one L2; a slice walks
// its groups one by one.  Fewer groups run in one linear order over all XCDs.
template <class T>
__device__ __forceinline__ void sgpr_ready(T x) {
  asm volatile("" ::"s"(x));
}

template <int D, bool QKN>
__global__ __launch_bounds__(kPThreads) void prefill_attn_kernel(PrefillArgs a) {
  __shared__ __align__(16) _Float16 smem[PrefillLds<D>::HALVES];
  // Every launch argument the prologue needs, in scalar registers before
  // anything else: one batch of kernel-argument loads (one round trip)
  // instead of batches issued as the code first needs them.
  sgpr_ready(a.q), sgpr_ready(a.kc), sgpr_ready(a.vc), sgpr_ready(a.cos_t);
  sgpr_ready(a.sin_t), sgpr_ready(a.layer0), sgpr_ready(a.n_launch_layers);
  sgpr_ready(a.n_heads), sgpr_ready(a.n_kv_heads), sgpr_ready(a.max_seq_len);
  sgpr_ready(a.rope_type), sgpr_ready(a.start_pos), sgpr_ready(a.n_tokens), sgpr_ready(a.bq);
  sgpr_ready(a.n_qblk), sgpr_ready(a.xcd_slices), sgpr_ready(a.groups_per_xcd);
  sgpr_ready(a.qb_major), sgpr_ready(a.paired), sgpr_ready(a.split_tiles);
  sgpr_ready(a.chunks_per_group), sgpr_ready(a.score_scale);
  if (QKN) sgpr_ready(a.qn);
  const int nq = a.n_qblk;
  // XCD slices (xcd_slices = 8), or one linear order when there are too few
  // groups to give every XCD its own (xcd_slices = 1)
  const int xcd = (int)(blockIdx.x % a.xcd_slices), l = (int)(blockIdx.x / a.xcd_slices);
  if (a.split_tiles > 0) {
    // chunks of split_tiles tiles: a group's chunks, heaviest q block first,
    // are consecutive workgroups of its XCD slice and consecutive slots
    const int cpg = a.chunks_per_group;
    const int group = xcd * a.groups_per_xcd + l / cpg;
    if (group >= a.n_launch_layers * a.n_kv_heads) return;
    const int r0 = l % cpg;
    int r = r0, qb = nq - 1;
    for (;; --qb) {
      const int nc = (prefill_unit_tiles(a, qb) + a.split_tiles - 1) / a.split_tiles;
      if (r < nc || qb == 0) {
        const int slot = nc > 1 ? group * cpg + r0 : -1;
        prefill_attn_unit<D, QKN>(a, smem, group, qb, r * a.split_tiles, (r + 1) * a.split_tiles,
                                  slot);
        return;
      }
      r -= nc;
    }
  }
  if (!a.paired) {
    int group, qb;
    if (a.qb_major) {
      group = xcd * a.groups_per_xcd + l % a.groups_per_xcd;
      qb = nq - 1 - l / a.groups_per_xcd;
    } else {
      group = xcd * a.groups_per_xcd + l / nq;
      qb = nq - 1 - l % nq;
    }
    if (group >= a.n_launch_layers * a.n_kv_heads) return;
    prefill_attn_unit<D, QKN>(a, smem, group, qb, 0, INT_MAX, -1);
    return;
  }
  const int np = (nq + 1) / 2;
  const int group = xcd * a.groups_per_xcd + l / np;
  const int p = l % np;
  if (group >= a.n_launch_layers * a.n_kv_heads) return;
  prefill_attn_unit<D, QKN>(a, smem, group, nq - 1 - p, 0, INT_MAX, -1);
  // the unit's last barrier follows every wave's last LDS read: the next
  // unit may refill the buffers
  if (p != nq - 1 - p) prefill_attn_unit<D, QKN>(a, smem, group, p, 0, INT_MAX, -1);
}

// K-split workgroups for launches of a few units (one layer of a whole
// prompt: fewer units than CUs): KS groups of 4 waves share each unit's
// tiles, so a group takes ~1/KS of the heaviest unit's tiles; units in
// heaviest-first order.  LDS: KS tile buffers, reused for the groups' merge.
template <int D, int KS>
struct KsplitLds {
  static constexpr size_t kTiles = (size_t)KS * PrefillLds<D>::HALVES * 2;
  static constexpr size_t kMerge = (size_t)(KS - 1) * kPCols * (D + 4) * 4;
  static constexpr size_t kStage = (size_t)PrefillLds<D>::QSTAGE * 2;
  static constexpr size_t kTM = kTiles > kMerge ? kTiles : kMerge;
  static constexpr size_t kBytes = kTM > kStage ? kTM : kStage;
};
template <int D, bool QKN, int KS>
__global__ __launch_bounds__(kPThreads * KS) void prefill_attn_ksplit_kernel(PrefillArgs a) {
  __shared__ __align__(16) _Float16 smem[KsplitLds<D, KS>::kBytes / 2];
  sgpr_ready(a.q), sgpr_ready(a.kc), sgpr_ready(a.vc), sgpr_ready(a.cos_t);
  sgpr_ready(a.sin_t), sgpr_ready(a.layer0), sgpr_ready(a.n_launch_layers);
  sgpr_ready(a.n_heads), sgpr_ready(a.n_kv_heads), sgpr_ready(a.max_seq_len);
  sgpr_ready(a.rope_type), sgpr_ready(a.start_pos), sgpr_ready(a.n_tokens), sgpr_ready(a.bq);
  sgpr_ready(a.n_qblk), sgpr_ready(a.score_scale);
  if (QKN) sgpr_ready(a.qn);
  const int n_groups = a.n_launch_layers * a.n_kv_heads;
  const int l = (int)blockIdx.x;
  const int qb = a.n_qblk - 1 - l / n_groups, group = l % n_groups;
  if (qb < 0) return;
  prefill_attn_unit<D, QKN, KS>(a, smem, group, qb, 0, INT_MAX, -1);
}

// Combines the chunks of split units, one thread per (unit, column, 4 output
// elements); units with a single chunk wrote their output directly.  Per
// column: M = max of the chunks' maxima, out = sum 2^(m-M) O / sum 2^(m-M) l
// (chunk 0 holds row 0, which every column sees, so M is finite).  The
// chunks' loads are independent, so each thread waits about twice.
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  constexpr int Q = D / 4;
  const int nq = a.n_qblk;
  const long item = (long)blockIdx.x * 256 + threadIdx.x;
  const int unit = (int)(item / (kPCols * Q));
  if (unit >= a.n_launch_layers * a.n_kv_heads * nq) return;
  const int group = unit / nq, qb = unit % nq;
  const int c = (int)(item / Q % kPCols), q4 = (int)(item % Q);
  const int G = a.n_heads / a.n_kv_heads;
  const int tok = c / G, hh = c % G;
  const int i0 = qb * a.bq;
  const int T = a.split_tiles;
  const int nc = (prefill_unit_tiles(a, qb) + T - 1) / T;
  if (nc <= 1 || tok >= a.bq || i0 + tok >= a.n_tokens) return;
  int first = 0;  // the unit's first slot within its group's list (heaviest first)
  for (int q = nq - 1; q > qb; --q) first += (prefill_unit_tiles(a, q) + T - 1) / T;
  const size_t pc0 = ((size_t)group * a.chunks_per_group + first) * kPCols + c;
  float M = -INFINITY;
  for (int k = 0; k < nc; ++k) M = fmaxf(M, a.part_m[pc0 + (size_t)k * kPCols]);
  float L = 0.f;
  float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k = 0; k < nc; ++k) {
    const size_t pc = pc0 + (size_t)k * kPCols;
    const float w = fast_exp2(a.part_m[pc] - M);
    const float4 po = *(const float4*)(a.part_o + pc * D + 4 * q4);
    L += w * a.part_l[pc];
    O.x += w * po.x, O.y += w * po.y, O.z += w * po.z, O.w += w * po.w;
  }
  const float inv = 1.0f / L;
  const int kvh = group % a.n_kv_heads, li = group / a.n_kv_heads;
  float* orow = a.out + ((size_t)li * a.n_tokens + i0 + tok) * a.out_stride +
                (size_t)(kvh * G + hh) * D;
  *(float4*)(orow + 4 * q4) = make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
}

}  // namespace

namespace plh {
// plh_set_tuning key 5: prefill chunking of small launches (0 automatic, -1
// never, or a fixed chunk of 2, 4, 8 or 16 tiles)
int g_prefill_split = 0;
// plh_set_tuning key 6: K-split workgroups (0 automatic, -1 never, 2 or 3
// groups of 4 waves; 3 only for head_dim 64)
int g_prefill_ksplit = 0;
}  // namespace plh

static int attn_prefill_impl(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                             int max_seq_len, int rope_type, int layer0, int n_launch_layers,
                             int start_pos, int n_tokens, const float* q, const float* k,
                             const float* v, uint16_t* key_cache, uint16_t* val_cache,
                             const float* rope_cos, const float* rope_sin, float* out,
                             int out_stride, const float* q_norm, const float* k_norm,
                             float norm_eps) {
  Context& c = ctx();
  if (!c.stream) {
    set_error("plh_attn_prefill: library not initialised");
    return -1;
  }
  if (head_dim < 2 || head_dim > 256 || head_dim % 2) {
    set_error("plh_attn_prefill: head_dim %d not supported (even, at most 256)", head_dim);
    return -1;
  }
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads) {
    set_error("plh_attn_prefill: n_heads %d must be a multiple of n_kv_heads %d", n_heads,
              n_kv_heads);
    return -1;
  }
  const int G = n_heads / n_kv_heads;
  if (rope_type != PLH_ROPE_LLAMA && rope_type != PLH_ROPE_QWEN) {
    set_error("plh_attn_prefill: unknown rope_type %d", rope_type);
    return -1;
  }
  if (max_seq_len <= 0 || start_pos < 0 || n_tokens < 0 ||
      (long)start_pos + (long)n_tokens > (long)max_seq_len) {
    set_error("plh_attn_prefill: rows [%d, %ld) outside [0, %d)", start_pos,
              (long)start_pos + n_tokens, max_seq_len);
    return -1;
  }
  if (layer0 < 0 || n_launch_layers <= 0 || layer0 + n_launch_layers > n_layers) {
    set_error("plh_attn_prefill: layers [%d, %d) outside [0, %d)", layer0,
              layer0 + n_launch_layers, n_layers);
    return -1;
  }
  if (out_stride < n_heads * head_dim) {
    set_error("plh_attn_prefill: out_stride %d must be >= n_heads*head_dim %d", out_stride,
              n_heads * head_dim);
    return -1;
  }
  if ((q_norm == nullptr) != (k_norm == nullptr)) {
    set_error("plh_attn_prefill_qknorm: q_norm and k_norm must both be given or both be null");
    return -1;
  }
  if (n_tokens == 0) return 0;
  if (!q || !k || !v || !key_cache || !val_cache || !rope_cos || !rope_sin || !out) {
    set_error("plh_attn_prefill: null pointer");
    return -1;
  }
  const bool qkn = q_norm != nullptr;
  // The tuned kernels take head_dim 64 / 128, a GQA group that fits one
  // workgroup's columns and 16-byte output rows; everything else the
  // reference accepts runs on the generic kernels.
  if ((head_dim != 64 && head_dim != 128) || G > kPCols || out_stride % 4)
    return attn_generic(n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
                        n_launch_layers, start_pos, n_tokens, q, k, v, key_cache, val_cache,
                        rope_cos, rope_sin, out, out_stride, q_norm, k_norm, norm_eps, nullptr,
                        nullptr);

  PrefillArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.kc = key_cache;
  a.vc = val_cache;
  a.cos_t = rope_cos;
  a.sin_t = rope_sin;
  a.out = out;
  a.layer0 = layer0;
  a.n_launch_layers = n_launch_layers;
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.max_seq_len = max_seq_len;
  a.rope_type = rope_type;
  a.start_pos = start_pos;
  a.n_tokens = n_tokens;
  a.out_stride = out_stride;
  a.bq = kPCols / G;
  a.n_qblk = (n_tokens + a.bq - 1) / a.bq;
  const int n_groups = n_launch_layers * n_kv_heads;
  a.n_units = n_groups * a.n_qblk;
  // XCD slices need enough groups to keep all eight XCDs busy
  a.xcd_slices = n_groups >= 32 ? 8 : 1;
  a.groups_per_xcd = (n_groups + a.xcd_slices - 1) / a.xcd_slices;
  // pairs of q blocks when the launch holds many rounds of workgroups (long
  // prompts, wide models); single blocks, heaviest first, otherwise
  const long slots = 3L * (c.num_cus > 0 ? c.num_cus : 256);
  a.paired = a.n_qblk >= 4 && a.n_units >= 8 * slots ? 1 : 0;
  a.per_xcd = a.groups_per_xcd * (a.paired ? (a.n_qblk + 1) / 2 : a.n_qblk);
  // Launches with few q blocks (one layer of a prompt chunk, or of a short
  // or narrow prompt: at most a quarter as many blocks as CUs) split their
  // blocks into chunks of T tiles, merged afterwards: the heaviest block is
  // the critical path.  Blocks of more than 8 tiles are split; T is the
  // smallest of 2, 4, 8 whose chunks still fit one per CU, else 8.  Measured on one-layer launches: 128 tokens at start
  // 1024 (T = 8), TinyLlama 32 -> 23 us, Llama-2 51 -> 32 us; Qwen3 512
  // tokens from 0 (T = 4), 820 -> 790 us per 28-layer step against T = 8;
  // launches with more blocks lose to the extra prologues and the merge.
  a.split_tiles = 0;
  a.chunks_per_group = 0;
  if (!a.paired && g_prefill_split >= 0) {
    const int max_tiles = prefill_unit_tiles(a, a.n_qblk - 1);
    const int cus = c.num_cus > 0 ? c.num_cus : 256;
    auto chunks_of = [&](int T) {
      int cpg = 0;
      for (int qb = 0; qb < a.n_qblk; ++qb) cpg += (prefill_unit_tiles(a, qb) + T - 1) / T;
      return cpg;
    };
    int pick = 0, pick_cpg = 0;
    if (g_prefill_split > 0) {
      if (max_tiles > g_prefill_split) pick = g_prefill_split;
    } else if ((long)a.n_units * 4 <= cus && max_tiles > 8) {
      for (int T = 2; T < 8 && !pick; T *= 2)
        if ((long)n_groups * chunks_of(T) <= cus) pick = T;
      if (!pick) pick = 8;
    }
    if (pick) pick_cpg = chunks_of(pick);
    if (pick) {
      const size_t n_slots = (size_t)n_groups * pick_cpg;
      const size_t po = n_slots * kPCols * head_dim * sizeof(float);
      const size_t pm = n_slots * kPCols * sizeof(float);
      if (ensure_workspace(po + 2 * pm)) return -1;
      a.split_tiles = pick;
      a.chunks_per_group = pick_cpg;
      a.part_o = (float*)c.ws;
      a.part_m = (float*)((char*)c.ws + po);
      a.part_l = (float*)((char*)c.ws + po + pm);
      a.per_xcd = a.groups_per_xcd * pick_cpg;
    }
  }
  // Launches of more blocks than that but at most one per CU (one layer of a
  // whole prompt) run each block in one K-split workgroup: 2 groups of 4
  // waves share its tiles and merge in LDS.  The groups share the CU's
  // SIMDs, so a tile costs a group more than a lone one: one-layer launches
  // of 512 tokens measured TinyLlama 16.3 -> 14.8 us (3 groups: 15.3),
  // Llama-2 1024 tokens 46.1 -> 40.6 us.  3 groups only when forced, and
  // only for head_dim 64 (head_dim 128 has registers for 2 waves per SIMD).
  int ksplit = 0;
  if (!a.paired && a.split_tiles == 0 && g_prefill_ksplit >= 0) {
    const int cus = c.num_cus > 0 ? c.num_cus : 256;
    const int kmax = head_dim == 64 ? 3 : 2;
    if (g_prefill_ksplit > 0)
      ksplit = g_prefill_ksplit < kmax ? g_prefill_ksplit : kmax;
    else if ((long)a.n_units * 4 > cus && a.n_units <= cus &&
             prefill_unit_tiles(a, a.n_qblk - 1) >= 4)
      ksplit = 2;
  }
  // K/V bytes one XCD slice reads: by q-block order when they fit in a
  // comfortable share of the XCD's 4 MB L2
  const double slice_kv = (double)a.groups_per_xcd * (start_pos + n_tokens) * head_dim * 2 * 2;
  a.qb_major = slice_kv <= 2.0 * 1024 * 1024 ? 1 : 0;
  a.qn = q_norm;
  a.kn = k_norm;
  a.norm_eps = norm_eps;
  a.score_scale = kLog2e / sqrtf((float)head_dim);

  const long groups = (long)n_launch_layers * n_tokens * n_kv_heads * (head_dim / 8);
  a.app32 = groups < (1L << 31) ? 1 : 0;
  a.fd_app_kvh = make_fastdiv((uint32_t)n_kv_heads);
  a.fd_app_tok = make_fastdiv((uint32_t)n_tokens);
  long ab = (groups + 255) / 256;
  if (ab > 16384) ab = 16384;
  const unsigned grid = (unsigned)(a.xcd_slices * a.per_xcd);
  const dim3 ag((unsigned)ab), ab256(256), pg(grid), pb(kPThreads);
  if (head_dim == 64) {
    if (qkn)
      hipLaunchKernelGGL((prefill_append_kernel<64, true>), ag, ab256, 0, c.stream, a);
    else
      hipLaunchKernelGGL((prefill_append_kernel<64, false>), ag, ab256, 0, c.stream, a);
  } else {
    if (qkn)
      hipLaunchKernelGGL((prefill_append_kernel<128, true>), ag, ab256, 0, c.stream, a);
    else
      hipLaunchKernelGGL((prefill_append_kernel<128, false>), ag, ab256, 0, c.stream, a);
  }
  if (check_hip(hipGetLastError(), "prefill_append_kernel")) return -1;
  if (ksplit > 0) {
    const dim3 kg((unsigned)a.n_units), kb((unsigned)(kPThreads * ksplit));
    if (head_dim == 64 && ksplit == 3) {
      if (qkn)
        hipLaunchKernelGGL((prefill_attn_ksplit_kernel<64, true, 3>), kg, kb, 0, c.stream, a);
      else
        hipLaunchKernelGGL((prefill_attn_ksplit_kernel<64, false, 3>), kg, kb, 0, c.stream, a);
    } else if (head_dim == 64) {
      if (qkn)
        hipLaunchKernelGGL((prefill_attn_ksplit_kernel<64, true, 2>), kg, kb, 0, c.stream, a);
      else
        hipLaunchKernelGGL((prefill_attn_ksplit_kernel<64, false, 2>), kg, kb, 0, c.stream, a);
    } else {
      if (qkn)
        hipLaunchKernelGGL((prefill_attn_ksplit_kernel<128, true, 2>), kg, kb, 0, c.stream, a);
      else
        hipLaunchKernelGGL((prefill_attn_ksplit_kernel<128, false, 2>), kg, kb, 0, c.stream, a);
    }
    return check_hip(hipGetLastError(), "prefill_attn_ksplit_kernel");
  }
  if (head_dim == 64) {
    if (qkn)
      hipLaunchKernelGGL((prefill_attn_kernel<64, true>), pg, pb, 0, c.stream, a);
    else
      hipLaunchKernelGGL((prefill_attn_kernel<64, false>), pg, pb, 0, c.stream, a);
  } else {
    if (qkn)
      hipLaunchKernelGGL((prefill_attn_kernel<128, true>), pg, pb, 0, c.stream, a);
    else
      hipLaunchKernelGGL((prefill_attn_kernel<128, false>), pg, pb, 0, c.stream, a);
  }
  if (check_hip(hipGetLastError(), "prefill_attn_kernel")) return -1;
  if (a.split_tiles > 0) {
    const dim3 mg((unsigned)(((long)a.n_units * kPCols * (head_dim / 4) + 255) / 256)), mb(256);
    if (head_dim == 64)
      hipLaunchKernelGGL((prefill_merge_kernel<64>), mg, mb, 0, c.stream, a);
    else
      hipLaunchKernelGGL((prefill_merge_kernel<128>), mg, mb, 0, c.stream, a);
    return check_hip(hipGetLastError(), "prefill_merge_kernel");
  }
  return 0;
}

extern "C" int plh_attn_prefill(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                                int max_seq_len, int rope_type, int layer0, int n_launch_layers,
                                int start_pos, int n_tokens, const float* q, const float* k,
                                const float* v, uint16_t* key_cache, uint16_t* val_cache,
                                const float* rope_cos, const float* rope_sin, float* out,
                                int out_stride) {
  return attn_prefill_impl(n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, rope_type,
                           layer0, n_launch_layers, start_pos, n_tokens, q, k, v, key_cache,
                           val_cache, rope_cos, rope_sin, out, out_stride, nullptr, nullptr, 0.0f);
}

extern "C" int plh_attn_prefill_qknorm(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                                       int max_seq_len, int rope_type, int layer0,
                                       int n_launch_layers, int start_pos, int n_tokens,
                                       const float* q, const float* k, const float* v,
                                       uint16_t* key_cache, uint16_t* val_cache,
                                       const float* rope_cos, const float* rope_sin, float* out,
                                       int out_stride, const float* q_norm, const float* k_norm,
                                       float norm_eps) {
  return attn_prefill_impl(n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, rope_type,
                           layer0, n_launch_layers, start_pos, n_tokens, q, k, v, key_cache,
                           val_cache, rope_cos, rope_sin, out, out_stride, q_norm, k_norm,
                           norm_eps);
}
