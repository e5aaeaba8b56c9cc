// attn_common.h -- device helpers shared by the decode and prefill kernels.
//
// All HIP sources are compiled with -ffp-contract=off: the reference's
// arithmetic (picolm/Makefile:2, -std=c11) never fuses a multiply into an
// add, and the RoPE rotation and the fp16 rounding of the KV cache must be
// bit-identical to it.  Where a fused multiply-add is harmless it is written
// explicitly with __builtin_fmaf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

namespace plh {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1e30f;  // finite "minus infinity" of the online softmax

// fp32 -> fp16 bits with the reference's rounding (quant.c:41-78): half an
// fp16 ulp is added to the magnitude and the result truncated, i.e. round half
// AWAY from zero; fp32 subnormals become signed zero; magnitudes below 2^-25
// become signed zero; overflow gives +-inf; NaN gives sign|0x7E00.  The
// hardware conversion rounds to nearest even and would differ on exact ties.
__device__ __forceinline__ uint16_t f16_bits_rha(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sgn = (u >> 16) & 0x8000u;
  uint32_t mag = u & 0x7FFFFFFFu;
  uint32_t e32 = mag >> 23;
  if (e32 == 0u) return (uint16_t)sgn;
  if (e32 == 0xFFu) return (uint16_t)(sgn | 0x7C00u | ((mag & 0x7FFFFFu) ? 0x0200u : 0u));
  int e16 = (int)e32 - 112;
  if (e16 >= 31) return (uint16_t)(sgn | 0x7C00u);
  if (e16 >= 1) return (uint16_t)(sgn | (((mag - (112u << 23)) + 0x1000u) >> 13));
  if (e16 < -10) return (uint16_t)sgn;
  uint32_t sig = (mag & 0x7FFFFFu) | 0x800000u;
  uint32_t sh = (uint32_t)(14 - e16);
  return (uint16_t)(sgn | ((sig + (1u << (sh - 1u))) >> sh));
}

// fp16 bits -> fp32.  The hardware widening is exact for every non-NaN input,
// which is all the reference's fp16_to_fp32 (quant.c:11-39) does.
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, h);
  return (float)x;
}

// One RoPE rotation as the reference writes it (tensor.c:583-601):
// a' = a*c - b*s, b' = a*s + b*c, each product and sum rounded separately
// (the translation unit is built with -ffp-contract=off).
__device__ __forceinline__ void rope_rotate(float& a, float& b, float c, float s) {
  float t0 = a * c;
  float t1 = b * s;
  float t2 = a * s;
  float t3 = b * c;
  a = t0 - t1;
  b = t2 + t3;
}

// RoPE rotation of an operand that is only used in dot products (q): the
// same pairing and table entries, with each output one product and one
// fused multiply-add (within one fp32 rounding of the reference's
// four-product form; the cached k rows keep that exact form).
__device__ __forceinline__ void rope_rotate_fused(float& a, float& b, float c, float s) {
  const float a0 = a;
  a = __builtin_fmaf(a0, c, -(b * s));
  b = __builtin_fmaf(a0, s, b * c);
}

// Splits an fp32 value into fp16 hi + lo so that an fp16 MFMA over both parts
// reproduces the fp32 operand to ~2^-22 relative (hi keeps 11 bits, lo the
// next 11).  Values must be below 65504 in magnitude (q columns are brought
// there by q_range_scale).
__device__ __forceinline__ void split_hi_lo(float x, _Float16& hi, _Float16& lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

// Range of a q column for the fp16 split.  amax is the largest |element| of
// the column (NaN-propagating maximum).  Columns with amax >= 2^15 are
// multiplied by 2^-e, with e chosen so that the largest element lands in
// [2^14, 2^15): a change of exponent, exact for every element that stays a
// normal number, and elements it pushes below fp16's range are below 2^-38
// of the largest one.  The column's score is then (K . q 2^-e) 2^e, so 2^e
// goes into its score scale.  Returns 2^-e (1 for ordinary columns, so their
// arithmetic is unchanged); *up gets 2^e.  inf / NaN columns get a finite
// scale and stay inf / NaN, as in the reference's fp32 arithmetic.
__device__ __forceinline__ float q_range_scale(float amax, float* up) {
  const int ex = (int)((__float_as_uint(amax) >> 23) & 0xFFu) - 127;  // floor(log2 amax)
  const int e = ex >= 15 ? ex - 14 : 0;                                // 0 .. 114
  *up = __uint_as_float((uint32_t)(127 + e) << 23);
  return __uint_as_float((uint32_t)(127 - e) << 23);
}

// Same split for a pair of values (|x| below 65504, or below 131008 for the
// softmax weights, which are at most 2^16: round-toward-zero keeps hi finite
// at 65504 and lo takes the rest):
// hi = rtz(x) by the packed round-toward-zero conversion, lo = f16(x - hi) by
// two mixed-precision FMAs (f16 first operand, f32 addend, f16 result written
// into the low / high half of the register).  x - hi is exact, so hi + lo
// keeps ~22 bits.  Three instructions per pair.
__device__ __forceinline__ void split_pair_rtz(float x0, float x1, half2_t& hi, half2_t& lo) {
  const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x0, x1));
  uint32_t l;
  asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(l) : "v"(h), "v"(x0));
  asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "+v"(l)
      : "v"(h), "v"(x1));
  hi = __builtin_bit_cast(half2_t, h);
  lo = __builtin_bit_cast(half2_t, l);
}

// IEEE-754 maximum (NaN-propagating); lowers to v_maximum3_f32 on gfx950
// without the NaN-quieting moves that fmaxf needs.
__device__ __forceinline__ float vmax(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16).  Within each 16-lane group,
// lane i passes the address of 4 consecutive fp16 values: chunk i%4 of row
// i/4 of a 4 x 16 block.  Lane i receives column i of that block, rows 0..3.
__device__ __forceinline__ half4_t lds_read_tr4(const _Float16* p) {
  typedef __fp16 fp16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4;
  return __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)p));
}

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_f16, lane = 32*h + i: A = row i, k 8*h .. 8*h+7;
// B = column i, k 8*h .. 8*h+7; C / D = column i, rows 8*(v/4) + 4*h + v%4
// for v = 0..15.
__device__ __forceinline__ f32x16_t mfma32x32x16(half8_t a, half8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Kernel arguments in scalar registers at one point: an empty asm statement
// that takes them all as scalar operands makes the compiler issue their
// loads together, behind one wait.  Left alone, it loads an argument just
// before its first use, and every load that sits behind a branch or a
// computed index then costs a memory round trip of its own before the
// kernel's first real load is issued.  (One statement: a chain of them gets
// one load and one wait each.)
#define PLH_ARGS_NOW(...) __asm__ volatile("" ::__VA_ARGS__)

// Maximum over lanes l and l^16 (resp. l^32) with the gfx950 row-swap
// permutes: permlane16_swap(x, x) returns rows {0,0,2,2} and {1,1,3,3} of x
// (rows of 16 lanes), permlane32_swap(x, x) returns halves {0,0} and {1,1}, so
// the larger of the two results is the pairwise maximum.  No LDS round trip.
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// ---- QK-norm (Qwen3, model.c:807-817 / 1029-1037) ---------------------------
// The reference's rmsnorm (tensor.c:425-492) as its x86-64 build runs it
// (AVX2: quant.h:33-46): eight lane sums a[j] += x[i]*x[i] over i = j mod 8
// in increasing i (product and sum rounded separately), folded as
// ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)), then 1/sqrtf(ss/size + eps); the
// normalised value is (x*scale)*w.  Device division and square root are
// correctly rounded (HIP's default), as on the host, so k rows normalised
// here round to the same fp16 bits.
//
// Pair scheme: four lanes share a row; the lane with pair index p (0..3)
// forms the sums a[2p] and a[2p+1] itself, in the reference's element order;
// the fold then adds partner lanes' sums.  Floating addition is commutative,
// so "own + partner" is the same value in both lanes and every lane ends with
// the reference's exact scale.
template <int D>
__device__ __forceinline__ void rms_pair_sums(const float* x, int p, float& s0, float& s1) {
  s0 = 0.f;
  s1 = 0.f;
#pragma unroll
  for (int m = 0; m < D / 8; ++m) {
    const float2 v = *(const float2*)(x + 8 * m + 2 * p);
    s0 = s0 + v.x * v.x;
    s1 = s1 + v.y * v.y;
  }
}

// sum2(v) = v + (v of the lane with pair index p^2), sum1 likewise for p^1.
template <class Sum2, class Sum1>
__device__ __forceinline__ float rms_scale_pairs(float s0, float s1, int size, float eps,
                                                 Sum2 sum2, Sum1 sum1) {
  const float l0 = sum2(s0), l1 = sum2(s1);  // p even: a0+a4, a1+a5; p odd: a2+a6, a3+a7
  const float h0 = sum1(l0), h1 = sum1(l1);  // (a0+a4)+(a2+a6), (a1+a5)+(a3+a7)
  return 1.0f / sqrtf((h0 + h1) / (float)size + eps);
}

// Scale of the head row of this lane's column when the row is already in
// registers as MFMA operands (lane (col, grp) holds element
// 32*db + 8*grp + j in x[db][j]): every lane keeps the eight running sums
// a[j] and adds, in increasing element order, the square held by lane
// (col, g) -- no memory traffic, D/8 * 4 cross-lane reads per lane.
template <int D>
__device__ __forceinline__ float rms_scale_cols(const float (&x)[D / 32][8], int col, float eps) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sq = x[db][j] * x[db][j];
        acc[j] = acc[j] + __shfl(sq, col + 16 * g, 64);
      }
  const float l0 = acc[0] + acc[4], l1 = acc[1] + acc[5];
  const float l2 = acc[2] + acc[6], l3 = acc[3] + acc[7];
  return 1.0f / sqrtf(((l0 + l2) + (l1 + l3)) / (float)D + eps);
}

// The same scale for the 32x32 MFMA operand layout: lane (h, col) holds
// element 16*s + 8*h + j in x[s][j], its partner lane col + 32 - 64*h the
// other half of the row.  permlane32_swap hands every lane both halves'
// squares (r[0] from half 0, r[1] from half 1), which are elements 16*s + j
// and 16*s + 8 + j: added in that order, each running sum a[j] sees the
// row's elements in increasing order.
template <int D>
__device__ __forceinline__ float rms_scale_halves(const float (&x)[D / 16][8], float eps) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < D / 16; ++s)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sq = x[s][j] * x[s][j];
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(sq), __float_as_uint(sq),
                                                      false, false);
      acc[j] = acc[j] + __uint_as_float(r[0]);
      acc[j] = acc[j] + __uint_as_float(r[1]);
    }
  const float l0 = acc[0] + acc[4], l1 = acc[1] + acc[5];
  const float l2 = acc[2] + acc[6], l3 = acc[3] + acc[7];
  return 1.0f / sqrtf(((l0 + l2) + (l1 + l3)) / (float)D + eps);
}

// Pair sums across the four 16-lane rows of a wave (p = lane / 16, the MFMA
// operand layout): the gfx950 row-swap permutes return the values of both
// rows of a pair, so their sum is own + partner.
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Scale of row x for a lane in 16-lane row grp of the MFMA layout (all four
// lanes of a column pass the same row).
template <int D>
__device__ __forceinline__ float rms_scale_grp(const float* x, int grp, float eps) {
  float s0, s1;
  rms_pair_sums<D>(x, grp, s0, s1);
  return rms_scale_pairs(s0, s1, D, eps, add_xor32, add_xor16);
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

}  // namespace plh

namespace plh {

// ---- rmsnorm scale of a whole vector by one workgroup -----------------------
// tensor.c:425-492 in the reference's x86-64 AVX2 order: eight lane sums
// acc[j] += x[8i+j]^2 (product rounded, then sum) over i in increasing order,
// folded as ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)), the tail x[i]^2 for
// i >= 8*(n/8) added one by one, then 1/sqrtf(ss/n + eps).  The workgroup
// writes the squares to LDS transposed (chain j's squares contiguous, pitch
// rms_sq_pitch(n)), eight lanes run the chains with batched LDS reads, and
// every thread folds the eight sums itself, so all return the same scale.
// sq: 8 * rms_sq_pitch(n) floats of LDS (free again once this returns);
// red: 8 floats of LDS.  Every thread of the workgroup must call it.
__host__ __device__ inline int rms_sq_pitch(int n) { return (n / 8 + 3) / 4 * 4 + 4; }

// The eight chains and the fold, once every square x[8i+j]^2 of the vector
// sits at sq[j * pitch + i] (see rms_scale_block).
template <int NT>
__device__ __forceinline__ float rms_chain_fold(const float* x, int n, float eps, const float* sq,
                                                float* red) {
  const int tid = threadIdx.x;
  const int n8 = n / 8, pitch = rms_sq_pitch(n);
  __syncthreads();
  if (tid < 8) {
    const float* s = sq + tid * pitch;
    float acc = 0.0f;
    int i = 0;
    for (; i + 32 <= n8; i += 32) {
      float4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = *(const float4*)(s + i + 4 * k);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        acc = acc + v[k].x;
        acc = acc + v[k].y;
        acc = acc + v[k].z;
        acc = acc + v[k].w;
      }
    }
    for (; i < n8; ++i) acc = acc + s[i];
    red[tid] = acc;
  }
  __syncthreads();
  const float l0 = red[0] + red[4], l1 = red[1] + red[5];
  const float l2 = red[2] + red[6], l3 = red[3] + red[7];
  float ss = (l0 + l2) + (l1 + l3);
  for (int i = 8 * n8; i < n; ++i) ss = ss + x[i] * x[i];
  return 1.0f / sqrtf(ss / (float)n + eps);
}

template <int NT>
__device__ __forceinline__ float rms_scale_block(const float* x, int n, float eps, float* sq,
                                                 float* red) {
  const int tid = threadIdx.x;
  const int n8 = n / 8, pitch = rms_sq_pitch(n);
  for (int idx = tid; idx < 8 * n8; idx += NT) {
    const float v = x[idx];
    sq[(idx & 7) * pitch + (idx >> 3)] = v * v;
  }
  return rms_chain_fold<NT>(x, n, eps, sq, red);
}

// rms_scale_block split in two for callers that have other loads to issue:
// rms_prefetch loads this thread's elements x[tid + NT*k] (k < K, vectors of
// at most NT*K elements) into registers; rms_scale_prefetched squares them
// into LDS and finishes.  Loads issued between the two calls do not delay
// the squares (the x loads were issued first and complete first).
template <int NT, int K>
__device__ __forceinline__ void rms_prefetch(const float* x, int n, float (&xv)[K]) {
  const int lim = 8 * (n / 8);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int idx = threadIdx.x + NT * k;
    xv[k] = idx < lim ? x[idx] : 0.0f;
  }
}
template <int NT, int K>
__device__ __forceinline__ float rms_scale_prefetched(const float* x, int n, float eps,
                                                      const float (&xv)[K], float* sq,
                                                      float* red) {
  const int lim = 8 * (n / 8), pitch = rms_sq_pitch(n);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int idx = threadIdx.x + NT * k;
    if (idx < lim) sq[(idx & 7) * pitch + (idx >> 3)] = xv[k] * xv[k];
  }
  return rms_chain_fold<NT>(x, n, eps, sq, red);
}

}  // namespace plh
