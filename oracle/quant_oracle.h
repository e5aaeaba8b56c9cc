/*
 * quant_oracle.h -- CPU restatement of picolm's weight GEMV (the path that
 * gpu_try_matmul offloads): the fused dequantize + dot products of quant.c
 * for Q4_K, Q6_K and Q8_0 (and F32) rows, as the reference's x86-64 build
 * runs them (AVX2 + FMA paths, quant.c:340-352, 390-452, 517-582, 627-659),
 * and matmul's row loop (tensor.c:200-215).
 *
 * TEST INFRASTRUCTURE ONLY: tests/, the smoke entry and the bench's CPU leg
 * load it to check results against; the product never links or calls it.
 *
 * The AVX2 paths keep eight running sums (one per 256-bit lane) and reduce
 * them with hsum_avx2 (quant.h:33-46), which adds as
 * ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)); _mm256_fmadd_ps is one fused
 * multiply-add per lane (fmaf here).  Scalar expressions are not contracted
 * (-std=c11).  Every function here keeps exactly that order, so its result is
 * bit-identical to the reference's.
 *
 * Pinning (tests/test_oracle_gemv.py): bit-exact against the reference's own
 * vec_dot_* and dequantize_row_* compiled into oracle/_ref, over random
 * blocks of every field; against float64 dequantize-then-dot on the same
 * rows; special blocks (zero scales, extreme fp16 scales, all-max quants).
 */
#ifndef PICOLM_QUANT_ORACLE_H
#define PICOLM_QUANT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids, quant.h:49-63 */
#define ORC_TYPE_F32 0
#define ORC_TYPE_F16 1
#define ORC_TYPE_Q4_0 2
#define ORC_TYPE_Q8_0 8
#define ORC_TYPE_Q4_K 12
#define ORC_TYPE_Q6_K 14

/* Bytes of one row of n weights (quant.c:283-325); 0 for other types. */
size_t orc_row_bytes(int qtype, int n);

/* quant.c:390-515 (AVX2 path) */
float orc_vec_dot_q4_K(const void *row, const float *x, int n);
/* quant.c:517-625 (AVX2 path) */
float orc_vec_dot_q6_K(const void *row, const float *x, int n);
/* quant.c:627-659 (AVX2 path) */
float orc_vec_dot_q8_0(const void *row, const float *x, int n);
/* quant.c:340-352 (AVX2 path) */
float orc_vec_dot_f32(const void *row, const float *x, int n);

/* quant.c:96-128, 193-262 (Q4_K, Q6_K, Q8_0, Q4_0, F16, F32) */
void orc_dequantize_row(int qtype, const void *row, float *dst, int n);

/* tensor.c:200-215 with quant.c:713-730's dispatch: out[i] = dot(row i, x)
 * for i < d.  Returns -1 for a type without a fused dot product. */
int orc_matmul(float *out, const float *x, const void *W, int n, int d, int qtype);

/* orc_matmul with the rows split over n_threads threads like the reference's
 * matmul thread pool (tensor.c:217-236); bit-identical output. */
int orc_matmul_mt(float *out, const float *x, const void *W, int n, int d, int qtype,
                  int n_threads);

#ifdef __cplusplus
}
#endif

#endif
