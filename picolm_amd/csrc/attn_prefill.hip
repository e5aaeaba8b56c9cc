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
// Attention workgroup = (layer, kv head, block of bq prompt tokens).  Its 8
// waves own 16 "columns" each; a column is one (token, q head) pair of the
// block, so all q heads of the kv head's GQA group share every K/V tile.
// K/V tiles of 32 rows are staged in LDS (double-buffered, loaded by the
// whole workgroup), both row-major:
//   S^T[t][c] = K[t][:] . q_c      A = K rows (ds_read_b128), B = q_c hi/lo
//   O^T[d][c] += V^T[d][t] P^T[t][c]  A = V^T (two ds_read_b64_tr_b16), B = P hi/lo
// The two 16-row MFMA blocks of S^T read K rows in the order
// pi_rb(i) = 8*(i/4) + 4*rb + i%4, which leaves lane group g holding rows
// 8g..8g+7 of the tile: exactly the K slots of the PV product, so P never
// leaves registers; the transposing LDS read turns row-major V into the
// d-major A operand.  q and P are split into fp16 hi + lo parts (two MFMAs
// each), keeping the products at ~fp32 precision.
//
// Softmax bookkeeping per tile is kept short: the maximum is taken over raw
// scores and the 1/sqrt(D)*log2(e) scale is folded into the exp2 argument;
// the causal mask is applied only on tiles that cross a column's last row;
// the running maximum is raised (and O, l rescaled) only when a new score
// exceeds it by more than 2^kLazy, so weights stay below 2^kLazy.  The exp2
// argument is the ROUNDED scaled score minus the running maximum (no fused
// multiply-add): rounding is monotone, so no weight exceeds that of the row
// that set the maximum test, whatever the magnitude of the scores (a fused
// product could exceed the margin by its rounding error once the scores
// pass 2^27 and overflow exp2).  Weights stay at most 2^16 (2^kLazy below
// scores of 2^26).
#include <math.h>

#include "attn_common.h"
#include "picolm_hip.h"
#include "plh_internal.h"

using namespace plh;

namespace {

constexpr int kPW = 8;               // waves per attention workgroup
constexpr int kPThreads = 64 * kPW;
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
    const int g = (int)(idx % NG);
    const long rest = idx / NG;
    const int kvh = (int)(rest % a.n_kv_heads);
    const long lt = rest / a.n_kv_heads;
    const int tok = (int)(lt % a.n_tokens);
    const int li = (int)(lt / a.n_tokens);
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
    *(uint2*)(a.kc + out_row + e0) = pack(kh);
    *(uint2*)(a.kc + out_row + e1) = pack(kh + 4);
    *(uint2*)(a.vc + out_row + e0) = pack(vh);
    *(uint2*)(a.vc + out_row + e1) = pack(vh + 4);
  }
}

template <int D, bool QKN>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(D == 64 ? 6 : 4)))
void prefill_attn_kernel(PrefillArgs a) {
  constexpr int ND = D / 32;     // 32-wide d blocks of QK
  constexpr int NO = D / 16;     // 16-wide d blocks of PV
  constexpr int KP = D + 8;      // LDS pitch of a K row (halves)
  constexpr int VP = D + 16;     // LDS pitch of a V row (halves): the 4 rows of a
                                 // transposing read land in disjoint banks
  constexpr int KCH = kKT * D / 8;  // 16-byte chunks of a K (or V) tile
  constexpr int KBUF = kKT * KP;  // one K tile buffer (halves)
  constexpr int VBUF = kKT * VP;  // one V tile buffer (halves)
  constexpr int VOFF = 2 * KBUF;  // V buffers follow the two K buffers
  __shared__ __align__(16) _Float16 smem[2 * KBUF + 2 * VBUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;

  // XCD-aware order: each XCD takes whole (layer, kv head) groups, so a
  // group's K/V tiles, read by all its q blocks, stay in one L2.  When the
  // slice's K/V fits in L2 its units run heaviest q block first across all
  // its groups (longest-first keeps the end of the launch even); otherwise
  // group by group, heaviest first within a group, so that each group's
  // tiles are reused while still cached.
  const int nq = a.n_qblk;
  const int xcd = (int)(blockIdx.x & 7), l = (int)(blockIdx.x >> 3);
  int group, qb;
  if (a.qb_major) {
    group = xcd * a.groups_per_xcd + l % a.groups_per_xcd;
    qb = nq - 1 - l / a.groups_per_xcd;
  } else {
    group = xcd * a.groups_per_xcd + l / nq;
    qb = nq - 1 - l % nq;
  }
  if (group >= a.n_launch_layers * a.n_kv_heads) return;
  const int kvh = group % a.n_kv_heads;
  const int li = group / a.n_kv_heads;
  const int layer = a.layer0 + li;
  const int G = a.n_heads / a.n_kv_heads;
  const int kv_dim = a.n_kv_heads * D;
  const int q_dim = a.n_heads * D;
  const int i0 = qb * a.bq;
  const int last_tok = min(i0 + a.bq, a.n_tokens) - 1;
  const int n_rows = a.start_pos + last_tok + 1;          // rows [0, n_rows) are needed
  const int n_tiles = (n_rows + kKT - 1) / kKT;

  // this lane's column: token i0+tok, q head kvh*G+hh
  const int c = wave * 16 + col;
  const int tok = c / G, hh = c - (c / G) * G;
  const bool cvalid = tok < a.bq && i0 + tok < a.n_tokens;
  const int tok_c = cvalid ? i0 + tok : last_tok;          // clamped for addressing
  const int p_col = a.start_pos + tok_c;                  // causal limit of the column
  // smallest causal limit among the wave's columns (wave-uniform)
  const int p_min = __builtin_amdgcn_readfirstlane(
      a.start_pos + min(i0 + (wave * 16) / G, last_tok));

  // ---- cooperative tile loads (issued early; stored to LDS after compute) --
  const size_t row0 = (size_t)layer * a.max_seq_len;
  const uint16_t* kbase = a.kc + row0 * kv_dim + (size_t)kvh * D;
  const uint16_t* vbase = a.vc + row0 * kv_dim + (size_t)kvh * D;
  constexpr int LPT = (2 * KCH + kPThreads - 1) / kPThreads;  // chunks per thread
  half8_t ld[LPT];
  auto issue_loads = [&](int t0) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int ch = tid + u * kPThreads;
      const int cc = ch % KCH;                 // chunk within its tile
      const int r = cc / (D / 8), q8 = cc % (D / 8);
      const int row = min(t0 + r, n_rows - 1);
      const uint16_t* src = (ch < KCH ? kbase : vbase) + (size_t)row * kv_dim + 8 * q8;
      ld[u] = *(const half8_t*)src;
    }
  };
  // LDS destination of each loaded chunk in buffer 0, and the step to buffer 1
  int st_off[LPT], st_step[LPT];
#pragma unroll
  for (int u = 0; u < LPT; ++u) {
    const int ch = tid + u * kPThreads;
    const int cc = ch % KCH;
    const int r = cc / (D / 8), q8 = cc % (D / 8);
    st_off[u] = ch < KCH ? r * KP + 8 * q8 : VOFF + r * VP + 8 * q8;
    st_step[u] = ch < KCH ? KBUF : VBUF;
  }
  auto store_lds = [&](int b) {
#pragma unroll
    for (int u = 0; u < LPT; ++u)
      if (tid + u * kPThreads < 2 * KCH)
        *(half8_t*)&smem[st_off[u] + b * st_step[u]] = ld[u];
  };
  issue_loads(0);

  // ---- q operands of this lane's column: rotated, split into fp16 hi + lo --
  // Columns past the prompt (cvalid false) read the last token's row and are
  // never stored; each column's softmax is independent, so they need no mask.
  half8_t qhi[ND], qlo[ND];
  float qup, qdown;  // 2^e and 2^-e of the column's range scale
  {
    const float* qrow = a.q + ((size_t)li * a.n_tokens + tok_c) * q_dim +
                        (size_t)(kvh * G + (cvalid ? hh : 0)) * D;
    const float* cr = a.cos_t + (size_t)p_col * (D / 2);
    const float* sr = a.sin_t + (size_t)p_col * (D / 2);
    float qf[ND][8];
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      const float4 x0 = *(const float4*)(qrow + 32 * db + 8 * grp);
      const float4 x1 = *(const float4*)(qrow + 32 * db + 8 * grp + 4);
      qf[db][0] = x0.x, qf[db][1] = x0.y, qf[db][2] = x0.z, qf[db][3] = x0.w;
      qf[db][4] = x1.x, qf[db][5] = x1.y, qf[db][6] = x1.z, qf[db][7] = x1.w;
    }
    if (QKN) {
      // QK-norm of the column's q head row before the rotation
      const float* wq = a.qn + (size_t)li * D;
      float w[ND][8];
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const float4 w0 = *(const float4*)(wq + 32 * db + 8 * grp);
        const float4 w1 = *(const float4*)(wq + 32 * db + 8 * grp + 4);
        w[db][0] = w0.x, w[db][1] = w0.y, w[db][2] = w0.z, w[db][3] = w0.w;
        w[db][4] = w1.x, w[db][5] = w1.y, w[db][6] = w1.z, w[db][7] = w1.w;
      }
      const float sc = rms_scale_cols<D>(qf, col, a.norm_eps);
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float t = qf[db][j] * sc;
          qf[db][j] = t * w[db][j];
        }
    }
    if (a.rope_type == PLH_ROPE_QWEN) {
#pragma unroll
      for (int db = 0; db < ND / 2; ++db)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int i = 32 * db + 8 * grp + j;
          rope_rotate_fused(qf[db][j], qf[db + ND / 2][j], cr[i], sr[i]);
        }
    } else {
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const float4 c4 = *(const float4*)(cr + 16 * db + 4 * grp);
        const float4 s4 = *(const float4*)(sr + 16 * db + 4 * grp);
        rope_rotate_fused(qf[db][0], qf[db][1], c4.x, s4.x);
        rope_rotate_fused(qf[db][2], qf[db][3], c4.y, s4.y);
        rope_rotate_fused(qf[db][4], qf[db][5], c4.z, s4.z);
        rope_rotate_fused(qf[db][6], qf[db][7], c4.w, s4.w);
      }
    }
    // the softmax scale log2(e)/sqrt(D) goes into q, so that the MFMA
    // produces scores in log2 units; then the column's range for the fp16
    // split (a power-of-two scale, undone on the scores: 1 unless some
    // |q| * scale >= 2^15)
    float amax = 0.f;
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        qf[db][j] *= a.score_scale;
        amax = vmax(amax, fabsf(qf[db][j]));
      }
    amax = max_xor32(max_xor16(amax));
    qdown = q_range_scale(amax, &qup);
#pragma unroll
    for (int db = 0; db < ND; ++db)
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        half2_t hi, lo;
        split_pair_rtz(qf[db][j] * qdown, qf[db][j + 1] * qdown, hi, lo);
        qhi[db][j] = hi[0], qhi[db][j + 1] = hi[1];
        qlo[db][j] = lo[0], qlo[db][j + 1] = lo[1];
      }
  }

  store_lds(0);
  __syncthreads();

  // Running maximum ms (log2 units) and the accumulators.  Each QK MFMA chain
  // starts from -ms (times the column's 2^-e), so it yields score - ms
  // directly; the maximum test and the exp2 then read the same values, which
  // keeps every weight bounded (<= 2^kLazy) whatever the scores' magnitude.
  // The first tile sets ms to its own maximum (row 0 is never masked).
  float ms = 0.f;
  float4_t negm = float4_t{0.f, 0.f, 0.f, 0.f};  // -ms * 2^-e, the QK accumulator start
  float4_t lsum = float4_t{0.f, 0.f, 0.f, 0.f};  // running sum (all 4 entries equal)
  const bool scaled_cols = __ballot(qup != 1.f) != 0;  // wave-uniform: rare
  half8_t ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = (_Float16)1.0f;
  float4_t o[NO];
#pragma unroll
  for (int ob = 0; ob < NO; ++ob) o[ob] = float4_t{0.f, 0.f, 0.f, 0.f};
  // transposing-read address of this lane: row 8*grp + col/4, chunk col%4
  const int vofs = (8 * grp + (col >> 2)) * VP + 4 * (col & 3);
  int kofs[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) kofs[rb] = (8 * (col >> 2) + 4 * rb + (col & 3)) * KP + 8 * grp;

  // one tile in buffer b (a constant at each call site, so the LDS offsets
  // fold into the instructions)
  auto tile = [&](const int b, const int it) {
    const int t0 = it * kKT;
    const bool more = it + 1 < n_tiles;
    if (more) issue_loads(t0 + kKT);

    // S^T - ms for this wave's 16 columns
    float4_t s[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      s[rb] = negm;
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const half8_t kk = *(const half8_t*)&smem[b * KBUF + kofs[rb] + 32 * db];
        s[rb] = mfma16x16x32(kk, qhi[db], s[rb]);
        s[rb] = mfma16x16x32(kk, qlo[db], s[rb]);
      }
    }
    // lane holds rows t0 + 8*grp + j, j = 4*rb + r
    float t[8];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) t[4 * rb + r] = s[rb][r];
    if (scaled_cols) {
#pragma unroll
      for (int j = 0; j < 8; ++j) t[j] *= qup;  // exact: a power of two
    }
    if (t0 + kKT - 1 > p_min) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (t0 + 8 * grp + j > p_col) t[j] = -INFINITY;
    }
    float tmax = t[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) tmax = vmax(tmax, t[j]);
    tmax = max_xor32(max_xor16(tmax));
    if (it == 0 || __ballot(tmax > kLazy)) {
      // first tile: ms = its maximum (nothing accumulated yet); later, raise
      // ms by the excess (columns at or below it keep theirs)
      const float d = it == 0 ? tmax : fmaxf(tmax, 0.f);
      if (it != 0) {
        const float alpha = fast_exp2(-d);
        lsum *= alpha;
#pragma unroll
        for (int ob = 0; ob < NO; ++ob) o[ob] *= alpha;
      }
      ms += d;
      const float nm = -ms * qdown;
      negm = float4_t{nm, nm, nm, nm};
#pragma unroll
      for (int j = 0; j < 8; ++j) t[j] -= d;
    }
    half8_t ph, pl;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      half2_t hi, lo;
      split_pair_rtz(fast_exp2(t[j]), fast_exp2(t[j + 1]), hi, lo);
      ph[j] = hi[0], ph[j + 1] = hi[1];
      pl[j] = lo[0], pl[j + 1] = lo[1];
    }
    // row sums on the matrix core: every row of ones . P^T is the column sum
    lsum = mfma16x16x32(ones, ph, lsum);
    lsum = mfma16x16x32(ones, pl, lsum);
#pragma unroll
    for (int ob = 0; ob < NO; ++ob) {
      const _Float16* vp = &smem[VOFF + b * VBUF + vofs + 16 * ob];
      const half4_t v0 = lds_read_tr4(vp);
      const half4_t v1 = lds_read_tr4(vp + 4 * VP);
      const half8_t va = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
      o[ob] = mfma16x16x32(va, ph, o[ob]);
      o[ob] = mfma16x16x32(va, pl, o[ob]);
    }

    if (more) store_lds(b ^ 1);
    __syncthreads();
  };
  for (int it = 0; it < n_tiles; it += 2) {
    tile(0, it);
    if (it + 1 < n_tiles) tile(1, it + 1);
  }

  // ---- normalise and write: lane holds d = 16*ob + 4*grp + r of its column ---
  if (cvalid) {
    const float inv = 1.0f / lsum[0];
    float* orow = a.out + ((size_t)li * a.n_tokens + i0 + tok) * a.out_stride +
                  (size_t)(kvh * G + hh) * D;
#pragma unroll
    for (int ob = 0; ob < NO; ++ob) {
      float4 w;
      w.x = o[ob][0] * inv;
      w.y = o[ob][1] * inv;
      w.z = o[ob][2] * inv;
      w.w = o[ob][3] * inv;
      *(float4*)(orow + 16 * ob + 4 * grp) = w;
    }
  }
}

}  // namespace

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
  if (head_dim != 64 && head_dim != 128) {
    set_error("plh_attn_prefill: head_dim %d not supported (64, 128)", head_dim);
    return -1;
  }
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads) {
    set_error("plh_attn_prefill: n_heads %d must be a multiple of n_kv_heads %d", n_heads,
              n_kv_heads);
    return -1;
  }
  const int G = n_heads / n_kv_heads;
  if (G > 16 * kPW) {
    set_error("plh_attn_prefill: GQA group %d larger than %d", G, 16 * kPW);
    return -1;
  }
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
  if (out_stride < n_heads * head_dim || out_stride % 4) {
    set_error("plh_attn_prefill: out_stride %d must be a multiple of 4 and >= n_heads*head_dim %d",
              out_stride, n_heads * head_dim);
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
  a.bq = (16 * kPW) / G;
  a.n_qblk = (n_tokens + a.bq - 1) / a.bq;
  const int n_groups = n_launch_layers * n_kv_heads;
  a.n_units = n_groups * a.n_qblk;
  a.groups_per_xcd = (n_groups + 7) / 8;
  a.per_xcd = a.groups_per_xcd * a.n_qblk;
  // K/V bytes one XCD slice reads: by q-block order when they fit in a
  // comfortable share of the XCD's 4 MB L2
  const double slice_kv = (double)a.groups_per_xcd * (start_pos + n_tokens) * head_dim * 2 * 2;
  a.qb_major = slice_kv <= 2.0 * 1024 * 1024 ? 1 : 0;
  a.qn = q_norm;
  a.kn = k_norm;
  a.norm_eps = norm_eps;
  a.score_scale = kLog2e / sqrtf((float)head_dim);

  const long groups = (long)n_launch_layers * n_tokens * n_kv_heads * (head_dim / 8);
  long ab = (groups + 255) / 256;
  if (ab > 16384) ab = 16384;
  const unsigned grid = (unsigned)(8 * a.per_xcd);
  const dim3 ag((unsigned)ab), ab256(256), pg(grid), pb(kPThreads);
  if (head_dim == 64 && !qkn) {
    hipLaunchKernelGGL((prefill_append_kernel<64, false>), ag, ab256, 0, c.stream, a);
    if (check_hip(hipGetLastError(), "prefill_append_kernel")) return -1;
    hipLaunchKernelGGL((prefill_attn_kernel<64, false>), pg, pb, 0, c.stream, a);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL((prefill_append_kernel<64, true>), ag, ab256, 0, c.stream, a);
    if (check_hip(hipGetLastError(), "prefill_append_kernel")) return -1;
    hipLaunchKernelGGL((prefill_attn_kernel<64, true>), pg, pb, 0, c.stream, a);
  } else if (!qkn) {
    hipLaunchKernelGGL((prefill_append_kernel<128, false>), ag, ab256, 0, c.stream, a);
    if (check_hip(hipGetLastError(), "prefill_append_kernel")) return -1;
    hipLaunchKernelGGL((prefill_attn_kernel<128, false>), pg, pb, 0, c.stream, a);
  } else {
    hipLaunchKernelGGL((prefill_append_kernel<128, true>), ag, ab256, 0, c.stream, a);
    if (check_hip(hipGetLastError(), "prefill_append_kernel")) return -1;
    hipLaunchKernelGGL((prefill_attn_kernel<128, true>), pg, pb, 0, c.stream, a);
  }
  return check_hip(hipGetLastError(), "prefill_attn_kernel");
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
