/*
 * attn_oracle.c -- CPU restatement of picolm's attention block (test oracle).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, the smoke entry and the bench's
 * CPU-baseline leg to check results against.  Never linked into the product
 * library.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off (oracle/Makefile).  The reference
 * builds with -O2 -std=c11 (picolm/Makefile:2), whose ISO mode disables FMA
 * contraction, so every product and sum below is individually rounded in the
 * order written.
 */
#ifndef _GNU_SOURCE
#define _GNU_SOURCE
#endif
#include "attn_oracle.h"

#include <math.h>
#include <pthread.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32                                                            */
/* ------------------------------------------------------------------------ */

/* quant.c:11-39.  Normal and special values rebias the exponent (15 -> 127)
 * and widen the mantissa; subnormals are m * 2^-24, which is exact in fp32.
 * Kept out of line on purpose: the reference calls it across translation
 * units (no LTO), and the CPU baseline should carry the same call cost. */
__attribute__((noinline)) float orc_f16_to_f32(uint16_t h) {
    uint32_t sgn = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t u;
    if (e == 31u) {
        u = sgn | 0x7F800000u | (m << 13);
    } else if (e != 0u) {
        u = sgn | ((e + 112u) << 23) | (m << 13);
    } else {
        float mag = (float)m * 0x1p-24f;
        return sgn ? -mag : mag;
    }
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* quant.c:41-78.  The reference adds half an fp16 ulp (bit 12) to the
 * magnitude and truncates, i.e. rounds half AWAY from zero (its comment says
 * "nearest even"; the code does not).  Here the addition is done on the
 * rebiased magnitude so that a mantissa carry propagates into the exponent by
 * itself; a carry out of exponent 30 lands exactly on 0x7C00 (inf), as in the
 * reference.  fp16-subnormal results shift the full significand right with a
 * half-up rounding bit; magnitudes below 2^-25 flush to signed zero. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    uint32_t sgn = (u >> 16) & 0x8000u;
    uint32_t mag = u & 0x7FFFFFFFu;
    uint32_t e32 = mag >> 23;
    if (e32 == 0u) return (uint16_t)sgn;                 /* +-0, f32 subnormal */
    if (e32 == 0xFFu)                                    /* inf / nan */
        return (uint16_t)(sgn | 0x7C00u | ((mag & 0x7FFFFFu) ? 0x0200u : 0u));
    int e16 = (int)e32 - 112;
    if (e16 >= 31) return (uint16_t)(sgn | 0x7C00u);     /* overflow */
    if (e16 >= 1) {
        uint32_t r = ((mag - (112u << 23)) + 0x1000u) >> 13;
        return (uint16_t)(sgn | r);
    }
    if (e16 < -10) return (uint16_t)sgn;                 /* below 2^-25 */
    uint32_t sig = (mag & 0x7FFFFFu) | 0x800000u;
    uint32_t sh = (uint32_t)(14 - e16);                  /* 14 .. 24 */
    return (uint16_t)(sgn | ((sig + (1u << (sh - 1u))) >> sh));
}

void orc_f32_to_f16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f16_to_f32(src[i]);
}

static uint64_t mix64(uint64_t x) {
    x ^= x >> 30;
    x *= 0xBF58476D1CE4E5B9ull;
    x ^= x >> 27;
    x *= 0x94D049BB133111EBull;
    x ^= x >> 31;
    return x;
}

typedef struct {
    uint64_t first, count, sum;
} csum_job;

static void *csum_worker(void *arg) {
    csum_job *j = (csum_job *)arg;
    uint64_t s = 0;
    for (uint64_t i = 0; i < j->count; i++) {
        uint64_t x = j->first + i;
        uint32_t bits = (uint32_t)x;
        float f;
        memcpy(&f, &bits, sizeof f);
        s += ((uint64_t)orc_f32_to_f16(f) + 1u) * (mix64(x) | 1u);
    }
    j->sum = s;
    return NULL;
}

uint64_t orc_f16_checksum(uint64_t first, uint64_t count, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    csum_job jobs[64];
    uint64_t per = count / (uint64_t)n_threads;
    uint64_t at = first;
    for (int t = 0; t < n_threads; t++) {
        jobs[t].first = at;
        jobs[t].count = (t == n_threads - 1) ? first + count - at : per;
        jobs[t].sum = 0;
        at += jobs[t].count;
    }
    int started = 0;
    for (int t = 1; t < n_threads; t++) {
        if (pthread_create(&th[t], NULL, csum_worker, &jobs[t]) != 0) break;
        started = t;
    }
    csum_worker(&jobs[0]);
    for (int t = started + 1; t < n_threads; t++) csum_worker(&jobs[t]);
    uint64_t total = jobs[0].sum;
    for (int t = 1; t < n_threads; t++) {
        if (t <= started) pthread_join(th[t], NULL);
        total += jobs[t].sum;
    }
    return total;
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                     */
/* ------------------------------------------------------------------------ */

/* model.c:545-556: theta = (float)pos / powf(base, (float)(2i) / (float)D),
 * then cosf(theta), sinf(theta).  Same libm calls, same operand order. */
void orc_rope_tables(float *cos_tab, float *sin_tab, int max_seq_len,
                     int head_dim, float freq_base) {
    int half = head_dim / 2;
    for (int p = 0; p < max_seq_len; p++) {
        for (int i = 0; i < half; i++) {
            float expo = (float)(2 * i) / (float)head_dim;
            float theta = (float)p / powf(freq_base, expo);
            size_t at = (size_t)p * (size_t)half + (size_t)i;
            cos_tab[at] = cosf(theta);
            sin_tab[at] = sinf(theta);
        }
    }
}

/* One rotation, written as the reference's statement pair (tensor.c:583-601
 * and 541-556): new_a = a*c - b*s ; new_b = a*s + b*c. */
static void rot_pair(float *a, float *b, float c, float s) {
    float x0 = *a, x1 = *b;
    float t0 = x0 * c;
    float t1 = x1 * s;
    float t2 = x0 * s;
    float t3 = x1 * c;
    *a = t0 - t1;
    *b = t2 + t3;
}

static void rope_heads(float *x, int n, int head_dim, const float *c,
                       const float *s, int rope_type) {
    int half = head_dim / 2;
    for (int h = 0; h < n; h++) {
        float *xh = x + (size_t)h * (size_t)head_dim;
        for (int i = 0; i < half; i++) {
            if (rope_type == ORC_ROPE_QWEN)
                rot_pair(&xh[i], &xh[i + half], c[i], s[i]);
            else
                rot_pair(&xh[2 * i], &xh[2 * i + 1], c[i], s[i]);
        }
    }
}

/* tensor.c:531-603: all q heads, then all kv heads. */
void orc_rope(float *q, float *k, int head_dim, int n_heads, int n_kv_heads,
              const float *cos_pos, const float *sin_pos, int rope_type) {
    rope_heads(q, n_heads, head_dim, cos_pos, sin_pos, rope_type);
    rope_heads(k, n_kv_heads, head_dim, cos_pos, sin_pos, rope_type);
}

/* ------------------------------------------------------------------------ */
/* QK-norm (Qwen3)                                                          */
/* ------------------------------------------------------------------------ */

/* tensor.c:425-492 as the reference builds on x86-64 with AVX2 (quant.h:33-46
 * defines PICOLM_AVX2 from __AVX2__, which -march=native sets on any AVX2
 * host): eight lane sums acc[j] += x[i]*x[i] over i = j mod 8 (product and
 * sum rounded separately), folded as ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))
 * (hsum_avx2), a scalar tail for size % 8, then
 * ss = 1/sqrtf(ss/size + eps) and out[i] = (x[i]*ss)*w[i]. */
void orc_rmsnorm(float *out, const float *x, const float *w, int size, float eps) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < size; i += 8)
        for (int j = 0; j < 8; j++) {
            float sq = x[i + j] * x[i + j];
            acc[j] = acc[j] + sq;
        }
    float l0 = acc[0] + acc[4], l1 = acc[1] + acc[5];
    float l2 = acc[2] + acc[6], l3 = acc[3] + acc[7];
    float a02 = l0 + l2, a13 = l1 + l3;
    float ss = a02 + a13;
    for (; i < size; i++) ss += x[i] * x[i];
    ss = 1.0f / sqrtf(ss / (float)size + eps);
    for (int k = 0; k < size; k++) {
        float t = x[k] * ss;
        out[k] = t * w[k];
    }
}

/* model.c:807-817 / 1029-1037: every q head and every k head normalised with
 * the layer's q / k weights (head_dim floats each). */
static void qk_norm(float *q, float *k, int n_heads, int n_kv_heads, int head_dim,
                    const float *qnw, const float *knw, float eps) {
    for (int h = 0; h < n_heads; h++)
        orc_rmsnorm(q + (size_t)h * head_dim, q + (size_t)h * head_dim, qnw, head_dim, eps);
    for (int h = 0; h < n_kv_heads; h++)
        orc_rmsnorm(k + (size_t)h * head_dim, k + (size_t)h * head_dim, knw, head_dim, eps);
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                */
/* ------------------------------------------------------------------------ */

static int dims_ok(int n_heads, int n_kv_heads, int head_dim) {
    if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0) return 0;
    if (head_dim > 256 || (head_dim & 1)) return 0;
    if (n_heads % n_kv_heads) return 0;
    return 1;
}

/* model.c:848-892 for one token at position `pos` of one layer.  For each q
 * head: score_t = (sequential fp32 sum of q[d]*K[t][d]) / sqrtf(D); the
 * online softmax keeps (max, sum, acc[D]) and branches exactly as the
 * reference does: a new maximum rescales by expf(old-new) and adds V with
 * weight 1, otherwise weight expf(score-max).  out = acc * (1/sum). */
static void attend_heads(int n_heads, int n_kv_heads, int head_dim,
                         int seq_len, int layer, int pos, const float *q,
                         const uint16_t *key_cache, const uint16_t *val_cache,
                         float *out, int h_begin, int h_end) {
    int kv_dim = n_kv_heads * head_dim;
    int group = n_heads / n_kv_heads;
    const uint16_t *kl = key_cache + (size_t)layer * (size_t)seq_len * (size_t)kv_dim;
    const uint16_t *vl = val_cache + (size_t)layer * (size_t)seq_len * (size_t)kv_dim;
    float scale_div = sqrtf((float)head_dim);
    float acc[256];
    for (int h = h_begin; h < h_end; h++) {
        const float *qh = q + (size_t)h * (size_t)head_dim;
        int kvh = h / group;
        float m = -1e30f;
        float l = 0.0f;
        for (int d = 0; d < head_dim; d++) acc[d] = 0.0f;
        for (int t = 0; t <= pos; t++) {
            size_t row = (size_t)t * (size_t)kv_dim + (size_t)kvh * (size_t)head_dim;
            const uint16_t *kt = kl + row;
            const uint16_t *vt = vl + row;
            float sc = 0.0f;
            for (int d = 0; d < head_dim; d++) sc += qh[d] * orc_f16_to_f32(kt[d]);
            sc /= scale_div;
            if (sc > m) {
                float corr = expf(m - sc);
                l = l * corr + 1.0f;
                for (int d = 0; d < head_dim; d++)
                    acc[d] = acc[d] * corr + orc_f16_to_f32(vt[d]);
                m = sc;
            } else {
                float w = expf(sc - m);
                l += w;
                for (int d = 0; d < head_dim; d++)
                    acc[d] += w * orc_f16_to_f32(vt[d]);
            }
        }
        float inv = 1.0f / l;
        float *oh = out + (size_t)h * (size_t)head_dim;
        for (int d = 0; d < head_dim; d++) oh[d] = acc[d] * inv;
    }
}

static void attend_one(int n_heads, int n_kv_heads, int head_dim,
                       int seq_len, int layer, int pos, const float *q,
                       const uint16_t *key_cache, const uint16_t *val_cache,
                       float *out) {
    attend_heads(n_heads, n_kv_heads, head_dim, seq_len, layer, pos, q,
                 key_cache, val_cache, out, 0, n_heads);
}

/* Head-parallel variant for the CPU baseline's upper bound: the q heads are
 * split over pthreads, each head's arithmetic unchanged (so the results are
 * bit-identical to attend_one).  The reference itself runs this loop on one
 * thread whatever its -j (tensor.c:190-254 parallelises only the matmuls). */
struct attend_job {
    int n_heads, n_kv_heads, head_dim, seq_len, layer, pos;
    const float *q;
    const uint16_t *kc, *vc;
    float *out;
    int h_begin, h_end;
};

static void *attend_worker(void *arg) {
    struct attend_job *j = (struct attend_job *)arg;
    attend_heads(j->n_heads, j->n_kv_heads, j->head_dim, j->seq_len, j->layer,
                 j->pos, j->q, j->kc, j->vc, j->out, j->h_begin, j->h_end);
    return NULL;
}

static int attend_mt(int n_heads, int n_kv_heads, int head_dim, int seq_len,
                     int layer, int pos, const float *q, const uint16_t *kc,
                     const uint16_t *vc, float *out, int n_threads) {
    if (n_threads > n_heads) n_threads = n_heads;
    if (n_threads <= 1) {
        attend_one(n_heads, n_kv_heads, head_dim, seq_len, layer, pos, q, kc, vc, out);
        return 0;
    }
    if (n_threads > 256) n_threads = 256;
    pthread_t tid[256];
    struct attend_job job[256];
    int started = 0;
    for (int t = 0; t < n_threads; t++) {
        job[t] = (struct attend_job){n_heads, n_kv_heads, head_dim, seq_len, layer, pos, q, kc,
                                     vc, out, n_heads * t / n_threads,
                                     n_heads * (t + 1) / n_threads};
        if (t == 0) continue;
        if (pthread_create(&tid[t], NULL, attend_worker, &job[t]) != 0) break;
        started = t;
    }
    attend_worker(&job[0]);
    for (int t = 1; t <= started; t++) pthread_join(tid[t], NULL);
    /* heads of threads that failed to start run here */
    for (int t = started + 1; t < n_threads; t++) attend_worker(&job[t]);
    return 0;
}

/* model.c:802-805 + 822-826: row `pos` of layer `layer` gets f16(k), f16(v). */
static void append_row(int n_kv_heads, int head_dim, int seq_len, int layer,
                       int pos, const float *k, const float *v,
                       uint16_t *key_cache, uint16_t *val_cache) {
    size_t kv_dim = (size_t)n_kv_heads * (size_t)head_dim;
    size_t at = ((size_t)layer * (size_t)seq_len + (size_t)pos) * kv_dim;
    for (size_t d = 0; d < kv_dim; d++) {
        key_cache[at + d] = orc_f32_to_f16(k[d]);
        val_cache[at + d] = orc_f32_to_f16(v[d]);
    }
}

int orc_attn_core(int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                  int layer, int pos, const float *q,
                  const uint16_t *key_cache, const uint16_t *val_cache,
                  float *out) {
    if (!dims_ok(n_heads, n_kv_heads, head_dim)) return -1;
    if (layer < 0 || pos < 0 || pos >= max_seq_len) return -1;
    attend_one(n_heads, n_kv_heads, head_dim, max_seq_len, layer, pos, q,
               key_cache, val_cache, out);
    return 0;
}

int orc_attn_decode(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                    int max_seq_len, int rope_type, int layer, int pos,
                    float *q, float *k, const float *v,
                    uint16_t *key_cache, uint16_t *val_cache,
                    const float *cos_tab, const float *sin_tab, float *out) {
    return orc_attn_decode_qkn(n_layers, n_heads, n_kv_heads, head_dim, max_seq_len,
                               rope_type, layer, pos, q, k, v, key_cache, val_cache,
                               cos_tab, sin_tab, out, NULL, NULL, 0.0f);
}

int orc_attn_decode_qkn(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                        int max_seq_len, int rope_type, int layer, int pos,
                        float *q, float *k, const float *v,
                        uint16_t *key_cache, uint16_t *val_cache,
                        const float *cos_tab, const float *sin_tab, float *out,
                        const float *q_norm, const float *k_norm, float eps) {
    if (!dims_ok(n_heads, n_kv_heads, head_dim)) return -1;
    if (layer < 0 || layer >= n_layers || pos < 0 || pos >= max_seq_len) return -1;
    if ((q_norm == NULL) != (k_norm == NULL)) return -1;
    if (q_norm) qk_norm(q, k, n_heads, n_kv_heads, head_dim, q_norm, k_norm, eps);
    size_t half = (size_t)(head_dim / 2);
    const float *c = cos_tab + (size_t)pos * half;
    const float *s = sin_tab + (size_t)pos * half;
    orc_rope(q, k, head_dim, n_heads, n_kv_heads, c, s, rope_type);
    append_row(n_kv_heads, head_dim, max_seq_len, layer, pos, k, v, key_cache,
               val_cache);
    attend_one(n_heads, n_kv_heads, head_dim, max_seq_len, layer, pos, q,
               key_cache, val_cache, out);
    return 0;
}

int orc_attn_decode_mt(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                       int max_seq_len, int rope_type, int layer, int pos,
                       float *q, float *k, const float *v,
                       uint16_t *key_cache, uint16_t *val_cache,
                       const float *cos_tab, const float *sin_tab, float *out,
                       int n_threads) {
    if (!dims_ok(n_heads, n_kv_heads, head_dim)) return -1;
    if (layer < 0 || layer >= n_layers || pos < 0 || pos >= max_seq_len) return -1;
    size_t half = (size_t)(head_dim / 2);
    const float *c = cos_tab + (size_t)pos * half;
    const float *s = sin_tab + (size_t)pos * half;
    orc_rope(q, k, head_dim, n_heads, n_kv_heads, c, s, rope_type);
    append_row(n_kv_heads, head_dim, max_seq_len, layer, pos, k, v, key_cache,
               val_cache);
    return attend_mt(n_heads, n_kv_heads, head_dim, max_seq_len, layer, pos, q,
                     key_cache, val_cache, out, n_threads);
}

int orc_attn_prefill(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                     int max_seq_len, int rope_type, int layer, int start_pos,
                     int n_tokens, float *q, float *k, const float *v,
                     uint16_t *key_cache, uint16_t *val_cache,
                     const float *cos_tab, const float *sin_tab,
                     float *out, int out_stride) {
    return orc_attn_prefill_qkn(n_layers, n_heads, n_kv_heads, head_dim, max_seq_len,
                                rope_type, layer, start_pos, n_tokens, q, k, v, key_cache,
                                val_cache, cos_tab, sin_tab, out, out_stride, NULL, NULL,
                                0.0f);
}

int orc_attn_prefill_qkn(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                         int max_seq_len, int rope_type, int layer, int start_pos,
                         int n_tokens, float *q, float *k, const float *v,
                         uint16_t *key_cache, uint16_t *val_cache,
                         const float *cos_tab, const float *sin_tab,
                         float *out, int out_stride,
                         const float *q_norm, const float *k_norm, float eps) {
    if (!dims_ok(n_heads, n_kv_heads, head_dim)) return -1;
    if (layer < 0 || layer >= n_layers || start_pos < 0 || n_tokens < 0) return -1;
    if ((q_norm == NULL) != (k_norm == NULL)) return -1;
    if ((long)start_pos + (long)n_tokens > (long)max_seq_len) return -1;
    size_t q_dim = (size_t)n_heads * (size_t)head_dim;
    size_t kv_dim = (size_t)n_kv_heads * (size_t)head_dim;
    size_t half = (size_t)(head_dim / 2);
    for (int bi = 0; bi < n_tokens; bi++) {
        int pos = start_pos + bi;
        float *qb = q + (size_t)bi * q_dim;
        float *kb = k + (size_t)bi * kv_dim;
        const float *vb = v + (size_t)bi * kv_dim;
        if (q_norm) qk_norm(qb, kb, n_heads, n_kv_heads, head_dim, q_norm, k_norm, eps);
        orc_rope(qb, kb, head_dim, n_heads, n_kv_heads,
                 cos_tab + (size_t)pos * half, sin_tab + (size_t)pos * half,
                 rope_type);
        append_row(n_kv_heads, head_dim, max_seq_len, layer, pos, kb, vb,
                   key_cache, val_cache);
        attend_one(n_heads, n_kv_heads, head_dim, max_seq_len, layer, pos, qb,
                   key_cache, val_cache, out + (size_t)bi * (size_t)out_stride);
    }
    return 0;
}

/* Head-parallel prefill (the CPU baseline's upper bound): the per-token
 * prologue of orc_attn_prefill_qkn for every row first, then each thread runs
 * attend_heads for its q heads over all tokens. */
struct prefill_job {
    int n_heads, n_kv_heads, head_dim, seq_len, layer, start_pos, n_tokens;
    const float *q;
    const uint16_t *kc, *vc;
    float *out;
    int out_stride, h_begin, h_end;
};

static void *prefill_worker(void *arg) {
    struct prefill_job *j = (struct prefill_job *)arg;
    size_t q_dim = (size_t)j->n_heads * (size_t)j->head_dim;
    for (int bi = 0; bi < j->n_tokens; bi++)
        attend_heads(j->n_heads, j->n_kv_heads, j->head_dim, j->seq_len, j->layer,
                     j->start_pos + bi, j->q + (size_t)bi * q_dim, j->kc, j->vc,
                     j->out + (size_t)bi * (size_t)j->out_stride, j->h_begin, j->h_end);
    return NULL;
}

int orc_attn_prefill_mt(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                        int max_seq_len, int rope_type, int layer, int start_pos,
                        int n_tokens, float *q, float *k, const float *v,
                        uint16_t *key_cache, uint16_t *val_cache,
                        const float *cos_tab, const float *sin_tab,
                        float *out, int out_stride,
                        const float *q_norm, const float *k_norm, float eps,
                        int n_threads) {
    if (!dims_ok(n_heads, n_kv_heads, head_dim)) return -1;
    if (layer < 0 || layer >= n_layers || start_pos < 0 || n_tokens < 0) return -1;
    if ((q_norm == NULL) != (k_norm == NULL)) return -1;
    if ((long)start_pos + (long)n_tokens > (long)max_seq_len) return -1;
    size_t q_dim = (size_t)n_heads * (size_t)head_dim;
    size_t kv_dim = (size_t)n_kv_heads * (size_t)head_dim;
    size_t half = (size_t)(head_dim / 2);
    for (int bi = 0; bi < n_tokens; bi++) {
        int pos = start_pos + bi;
        float *qb = q + (size_t)bi * q_dim;
        float *kb = k + (size_t)bi * kv_dim;
        if (q_norm) qk_norm(qb, kb, n_heads, n_kv_heads, head_dim, q_norm, k_norm, eps);
        orc_rope(qb, kb, head_dim, n_heads, n_kv_heads,
                 cos_tab + (size_t)pos * half, sin_tab + (size_t)pos * half, rope_type);
        append_row(n_kv_heads, head_dim, max_seq_len, layer, pos, kb,
                   v + (size_t)bi * kv_dim, key_cache, val_cache);
    }
    if (n_threads > n_heads) n_threads = n_heads;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    pthread_t tid[256];
    struct prefill_job job[256];
    int started = 0;
    for (int t = 0; t < n_threads; t++) {
        job[t] = (struct prefill_job){n_heads, n_kv_heads, head_dim, max_seq_len, layer,
                                      start_pos, n_tokens, q, key_cache, val_cache, out,
                                      out_stride, n_heads * t / n_threads,
                                      n_heads * (t + 1) / n_threads};
        if (t == 0) continue;
        if (pthread_create(&tid[t], NULL, prefill_worker, &job[t]) != 0) break;
        started = t;
    }
    prefill_worker(&job[0]);
    for (int t = 1; t <= started; t++) pthread_join(tid[t], NULL);
    /* heads of threads that failed to start run here */
    for (int t = started + 1; t < n_threads; t++) prefill_worker(&job[t]);
    return 0;
}
