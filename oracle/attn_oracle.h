/*
 * attn_oracle.h -- CPU restatement of picolm's attention block.
 *
 * TEST INFRASTRUCTURE ONLY.  Results are checked against it: tests/, the smoke
 * entry and the bench's CPU-baseline leg load it; the product (libpicolm_hip)
 * never links, calls or falls back to it.
 *
 * Every function restates the reference semantics in plain C11 and is compiled
 * with -std=c11 -ffp-contract=off (the reference's Makefile builds with
 * -O2 -std=c11, which in GCC's ISO mode forbids FMA contraction).
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   orc_f32_to_f16 / orc_f16_to_f32 : exhaustive sweep against the compiled
 *       reference quant.c (oracle/_ref) plus known-answer vectors.
 *   orc_rope_tables                 : bit-exact against the reference's table
 *       (model.c init_rope_tables reached through oracle/ref_harness.c) and
 *       closed-form invariants (row 0 = (1,0), cos^2+sin^2 ~ 1).
 *   orc_rope                        : bit-exact against reference tensor.c rope.
 *   orc_attn_decode                 : bit-exact against model_forward_ex driven
 *       by ref_harness.c; brute-force double softmax on tiny shapes.
 *   orc_attn_prefill                : KV bits and next-layer inputs bit-exact
 *       against model_forward_prefill; equals orc_attn_decode step by step.
 */
#ifndef PICOLM_ATTN_ORACLE_H
#define PICOLM_ATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* rope_type values, model.h:15-18 */
#define ORC_ROPE_LLAMA 0
#define ORC_ROPE_QWEN 1

/* quant.c:11-39 -- exact fp16 -> fp32 widening (incl. subnormals, inf, nan). */
float orc_f16_to_f32(uint16_t h);

/* quant.c:41-78 -- fp32 -> fp16 with round-half-AWAY-from-zero on the
 * magnitude, fp32 subnormals flushed to signed zero, NaN -> sign|0x7E00. */
uint16_t orc_f32_to_f16(float f);

void orc_f32_to_f16_array(const float *src, uint16_t *dst, size_t n);
void orc_f16_to_f32_array(const uint16_t *src, float *dst, size_t n);

/* Order-independent checksum of orc_f32_to_f16 over the fp32 bit patterns
 * [first, first + count): sum over x of (f16(x) + 1) * (mix64(x) | 1) mod 2^64.
 * Runs on n_threads pthreads. */
uint64_t orc_f16_checksum(uint64_t first, uint64_t count, int n_threads);

/* model.c:545-556 -- cos/sin tables [max_seq_len][head_dim/2], computed with
 * the host's libm powf/cosf/sinf in the reference's operation order. */
void orc_rope_tables(float *cos_tab, float *sin_tab, int max_seq_len,
                     int head_dim, float freq_base);

/* tensor.c:531-603 -- in-place rotation of q [n_heads*head_dim] and
 * k [n_kv_heads*head_dim] with one table row; LLaMA pairs (2i,2i+1),
 * QWEN pairs (i, i+head_dim/2).  Two rounded products and one rounded
 * add/sub per output (no FMA). */
void orc_rope(float *q, float *k, int head_dim, int n_heads, int n_kv_heads,
              const float *cos_pos, const float *sin_pos, int rope_type);

/* model.c:802-805, 819-892 -- one layer, one token:
 *   rope(q, k) in place, append f16(k), f16(v) at row `pos` of layer `layer`,
 *   online-softmax GQA attention over rows 0..pos, out [n_heads*head_dim].
 * Cache layout: cache[((layer*max_seq_len + t)*n_kv_heads + kvh)*head_dim + d].
 * Returns 0, or -1 if the arguments are out of range. */
int orc_attn_decode(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                    int max_seq_len, int rope_type, int layer, int pos,
                    float *q, float *k, const float *v,
                    uint16_t *key_cache, uint16_t *val_cache,
                    const float *cos_tab, const float *sin_tab, float *out);

/* orc_attn_decode with the q heads split over n_threads pthreads (each head's
 * arithmetic unchanged, so the output is bit-identical).  For the CPU
 * baseline's "head-parallel upper bound" only: the reference runs this loop
 * on one thread. */
int orc_attn_decode_mt(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                       int max_seq_len, int rope_type, int layer, int pos,
                       float *q, float *k, const float *v,
                       uint16_t *key_cache, uint16_t *val_cache,
                       const float *cos_tab, const float *sin_tab, float *out,
                       int n_threads);

/* model.c:1019-1090 -- one layer, n_tokens prompt rows starting at start_pos,
 * processed serially: rope, append, attention over rows 0..start_pos+bi.
 * q [n_tokens][n_heads*head_dim] and k [n_tokens][kv_dim] rotated in place,
 * v [n_tokens][kv_dim]; out row bi at out + bi*out_stride. */
int orc_attn_prefill(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                     int max_seq_len, int rope_type, int layer, int start_pos,
                     int n_tokens, float *q, float *k, const float *v,
                     uint16_t *key_cache, uint16_t *val_cache,
                     const float *cos_tab, const float *sin_tab,
                     float *out, int out_stride);

/* Qwen3 QK-norm variants (model.c:807-817 decode, 1029-1037 prefill): before
 * the rotation every q head is RMS-normalised with q_norm[head_dim] and every
 * k head with k_norm[head_dim] (epsilon eps).  q_norm = k_norm = NULL gives
 * the plain functions above; only one of them NULL is an error. */
int orc_attn_decode_qkn(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                        int max_seq_len, int rope_type, int layer, int pos,
                        float *q, float *k, const float *v,
                        uint16_t *key_cache, uint16_t *val_cache,
                        const float *cos_tab, const float *sin_tab, float *out,
                        const float *q_norm, const float *k_norm, float eps);
int orc_attn_prefill_qkn(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                         int max_seq_len, int rope_type, int layer, int start_pos,
                         int n_tokens, float *q, float *k, const float *v,
                         uint16_t *key_cache, uint16_t *val_cache,
                         const float *cos_tab, const float *sin_tab,
                         float *out, int out_stride,
                         const float *q_norm, const float *k_norm, float eps);

/* orc_attn_prefill_qkn with the attention split over n_threads pthreads by q
 * head (each thread walks every token for its heads).  QK-norm, rotation and
 * the appends run first, serially, for all n_tokens rows: each token's
 * attention reads only rows up to its own position, so the output and caches
 * are bit-identical to the serial function.  For the CPU baseline's
 * "head-parallel upper bound" only: the reference runs this loop on one
 * thread. */
int orc_attn_prefill_mt(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                        int max_seq_len, int rope_type, int layer, int start_pos,
                        int n_tokens, float *q, float *k, const float *v,
                        uint16_t *key_cache, uint16_t *val_cache,
                        const float *cos_tab, const float *sin_tab,
                        float *out, int out_stride,
                        const float *q_norm, const float *k_norm, float eps,
                        int n_threads);

/* tensor.c:425-492 rmsnorm in the reference's x86-64 AVX2 build order (see
 * the definition).  out may alias x. */
void orc_rmsnorm(float *out, const float *x, const float *w, int size, float eps);

/* Attention only (model.c:848-892 for one token): no rope, no append.  Used
 * by tests that pin the softmax itself on hand-made caches. */
int orc_attn_core(int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                  int layer, int pos, const float *q,
                  const uint16_t *key_cache, const uint16_t *val_cache,
                  float *out);

#ifdef __cplusplus
}
#endif

#endif
