/*
 * quant_oracle.c -- restatement of picolm's fused dequantize + dot products
 * (test oracle; see quant_oracle.h for what it follows and how it is pinned).
 *
 * Vector lanes are modelled as arrays of eight floats.  Block layouts follow
 * quant.h:66-125: Q4_K = {fp16 d, fp16 dmin, scales[12], qs[128]} (144 B),
 * Q6_K = {ql[128], qh[64], int8 scales[16], fp16 d} (210 B),
 * Q8_0 = {fp16 d, int8 qs[32]} (34 B); all little-endian, unaligned.
 */
#include "quant_oracle.h"

#include <math.h>
#include <pthread.h>
#include <string.h>

#include "attn_oracle.h"

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* hsum_avx2 (quant.h:33-46): 128-bit halves added lane-wise, then the upper
 * pair onto the lower pair, then element 1 onto element 0. */
static float hsum8(const float v[8]) {
    const float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
    const float b0 = a0 + a2, b1 = a1 + a3;
    return b0 + b1;
}

size_t orc_row_bytes(int qtype, int n) {
    switch (qtype) {
        case ORC_TYPE_F32: return (size_t)n * 4;
        case ORC_TYPE_F16: return (size_t)n * 2;
        case ORC_TYPE_Q4_0: return (size_t)(n / 32) * 18;
        case ORC_TYPE_Q8_0: return (size_t)(n / 32) * 34;
        case ORC_TYPE_Q4_K: return (size_t)(n / 256) * 144;
        case ORC_TYPE_Q6_K: return (size_t)(n / 256) * 210;
        default: return 0;
    }
}

/* get_scale_min_k4 (quant.c:82-91): the 6-bit scale and min of sub-block j
 * from the 12 packed bytes. */
static void q4k_scale_min(int j, const uint8_t *s, int *sc, int *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

float orc_vec_dot_q4_K(const void *row, const float *x, int n) {
    const uint8_t *blk = (const uint8_t *)row;
    float sumf = 0.0f;
    for (int i = 0; i < n / 256; i++, blk += 144) {
        const float d = orc_f16_to_f32(rd16(blk));
        const float dmin = orc_f16_to_f32(rd16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *q = blk + 16;
        const float *xp = x + (size_t)i * 256;
        for (int j = 0; j < 4; j++, q += 32, xp += 64) {
            int sc, mn;
            q4k_scale_min(2 * j, scales, &sc, &mn);
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            q4k_scale_min(2 * j + 1, scales, &sc, &mn);
            const float d2 = d * (float)sc, m2 = dmin * (float)mn;
            /* lane k of the four accumulators; two 16-byte steps l = 0, 16,
             * each two fused multiply-adds (bytes l..l+7, then l+8..l+15) */
            float qx1[8] = {0}, sx1[8] = {0}, qx2[8] = {0}, sx2[8] = {0};
            for (int l = 0; l < 32; l += 16) {
                for (int k = 0; k < 8; k++) {
                    const float xl0 = xp[l + k], xl1 = xp[l + 8 + k];
                    const float xh0 = xp[l + 32 + k], xh1 = xp[l + 40 + k];
                    qx1[k] = fmaf((float)(q[l + k] & 0x0F), xl0, qx1[k]);
                    qx1[k] = fmaf((float)(q[l + 8 + k] & 0x0F), xl1, qx1[k]);
                    sx1[k] = sx1[k] + (xl0 + xl1);
                    qx2[k] = fmaf((float)(q[l + k] >> 4), xh0, qx2[k]);
                    qx2[k] = fmaf((float)(q[l + 8 + k] >> 4), xh1, qx2[k]);
                    sx2[k] = sx2[k] + (xh0 + xh1);
                }
            }
            const float s_qx1 = hsum8(qx1), s_x1 = hsum8(sx1);
            const float s_qx2 = hsum8(qx2), s_x2 = hsum8(sx2);
            const float t0 = d1 * s_qx1, t1 = m1 * s_x1, t2 = d2 * s_qx2, t3 = m2 * s_x2;
            sumf = sumf + (((t0 - t1) + t2) - t3);
        }
    }
    return sumf;
}

/* The 6-bit value of element e (0..255) of a Q6_K block, before the -32
 * offset (quant.c:199-213): 128-element halves c, each with four 32-element
 * quarters taking the low / high nibble of ql[0..31] / ql[32..63] and bit
 * pairs 0, 2, 4, 6 of qh[0..31]. */
static int q6k_value(const uint8_t *blk, int e) {
    const int c = e / 128, r = e % 128, quarter = r / 32, l = r % 32;
    const uint8_t *ql = blk + 64 * c, *qh = blk + 128 + 32 * c;
    const int lo = (quarter & 1) ? ql[l + 32] : ql[l];
    const int nib = (quarter & 2) ? (lo >> 4) : (lo & 0x0F);
    return nib | (((qh[l] >> (2 * quarter)) & 3) << 4);
}

float orc_vec_dot_q6_K(const void *row, const float *x, int n) {
    const uint8_t *blk = (const uint8_t *)row;
    float sumf = 0.0f;
    for (int i = 0; i < n / 256; i++, blk += 210) {
        const float d = orc_f16_to_f32(rd16(blk + 208));
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float *xp = x + (size_t)i * 256;
        /* group j = elements 16j..16j+15: lanes k take (v[k]-32)*x[k] fused
         * onto (v[8+k]-32)*x[8+k] (quant.c:559-578), then one hsum */
        float sums[16];
        for (int j = 0; j < 16; j++) {
            float p[8];
            for (int k = 0; k < 8; k++) {
                const float fl = (float)q6k_value(blk, 16 * j + k) - 32.0f;
                const float fh = (float)q6k_value(blk, 16 * j + 8 + k) - 32.0f;
                p[k] = fmaf(fl, xp[16 * j + k], fh * xp[16 * j + 8 + k]);
            }
            sums[j] = hsum8(p);
        }
        for (int j = 0; j < 16; j++) {
            const float ds = d * (float)sc[j];
            sumf = sumf + ds * sums[j];
        }
    }
    return sumf;
}

float orc_vec_dot_q8_0(const void *row, const float *x, int n) {
    const uint8_t *blk = (const uint8_t *)row;
    float sumf = 0.0f;
    for (int i = 0; i < n / 32; i++, blk += 34) {
        const float d = orc_f16_to_f32(rd16(blk));
        const int8_t *qs = (const int8_t *)(blk + 2);
        const float *xp = x + (size_t)i * 32;
        float acc[8];
        for (int k = 0; k < 8; k++) {
            const float p0 = (float)qs[k] * xp[k];
            const float p1 = (float)qs[8 + k] * xp[8 + k];
            const float p2 = (float)qs[16 + k] * xp[16 + k];
            const float p3 = (float)qs[24 + k] * xp[24 + k];
            acc[k] = (p0 + p1) + (p2 + p3);
        }
        sumf = sumf + d * hsum8(acc);
    }
    return sumf;
}

float orc_vec_dot_f32(const void *row, const float *x, int n) {
    const float *w = (const float *)row;
    float a0[8] = {0}, a1[8] = {0};
    int i = 0;
    for (; i + 15 < n; i += 16)
        for (int k = 0; k < 8; k++) {
            a0[k] = fmaf(w[i + k], x[i + k], a0[k]);
            a1[k] = fmaf(w[i + 8 + k], x[i + 8 + k], a1[k]);
        }
    float both[8];
    for (int k = 0; k < 8; k++) both[k] = a0[k] + a1[k];
    float sum = hsum8(both);
    for (; i < n; i++) {
        const float p = w[i] * x[i];
        sum = sum + p;
    }
    return sum;
}

void orc_dequantize_row(int qtype, const void *row, float *dst, int n) {
    const uint8_t *blk = (const uint8_t *)row;
    switch (qtype) {
        case ORC_TYPE_F32:
            memcpy(dst, row, (size_t)n * 4);
            break;
        case ORC_TYPE_F16:
            for (int i = 0; i < n; i++) dst[i] = orc_f16_to_f32(rd16(blk + 2 * i));
            break;
        case ORC_TYPE_Q4_0: /* quant.c:236-252: {fp16 d, qs[16]}, low nibbles first */
            for (int i = 0; i < n / 32; i++, blk += 18) {
                const float d = orc_f16_to_f32(rd16(blk));
                for (int j = 0; j < 32; j++) {
                    const int nib = j < 16 ? (blk[2 + j] & 0x0F) : (blk[2 + j - 16] >> 4);
                    dst[32 * i + j] = d * ((float)nib - 8.0f);
                }
            }
            break;
        case ORC_TYPE_Q8_0:
            for (int i = 0; i < n / 32; i++, blk += 34) {
                const float d = orc_f16_to_f32(rd16(blk));
                for (int k = 0; k < 32; k++) dst[32 * i + k] = d * (float)(int8_t)blk[2 + k];
            }
            break;
        case ORC_TYPE_Q4_K:
            for (int i = 0; i < n / 256; i++, blk += 144) {
                const float d = orc_f16_to_f32(rd16(blk));
                const float dmin = orc_f16_to_f32(rd16(blk + 2));
                for (int j = 0; j < 4; j++) {
                    int sc, mn;
                    q4k_scale_min(2 * j, blk + 4, &sc, &mn);
                    const float d1 = d * (float)sc, m1 = dmin * (float)mn;
                    q4k_scale_min(2 * j + 1, blk + 4, &sc, &mn);
                    const float d2 = d * (float)sc, m2 = dmin * (float)mn;
                    const uint8_t *q = blk + 16 + 32 * j;
                    float *y = dst + 256 * i + 64 * j;
                    for (int l = 0; l < 32; l++) {
                        const float a = d1 * (float)(q[l] & 0x0F);
                        y[l] = a - m1;
                        const float b = d2 * (float)(q[l] >> 4);
                        y[32 + l] = b - m2;
                    }
                }
            }
            break;
        case ORC_TYPE_Q6_K:
            for (int i = 0; i < n / 256; i++, blk += 210) {
                const float d = orc_f16_to_f32(rd16(blk + 208));
                const int8_t *sc = (const int8_t *)(blk + 192);
                for (int e = 0; e < 256; e++) {
                    /* scale index (quant.c:210-214): 16-element groups */
                    const float ds = d * (float)sc[e / 16];
                    dst[256 * i + e] = ds * (float)(q6k_value(blk, e) - 32);
                }
            }
            break;
        default:
            break;
    }
}

int orc_matmul(float *out, const float *x, const void *W, int n, int d, int qtype) {
    float (*dot)(const void *, const float *, int);
    switch (qtype) {
        case ORC_TYPE_Q4_K: dot = orc_vec_dot_q4_K; break;
        case ORC_TYPE_Q6_K: dot = orc_vec_dot_q6_K; break;
        case ORC_TYPE_Q8_0: dot = orc_vec_dot_q8_0; break;
        case ORC_TYPE_F32: dot = orc_vec_dot_f32; break;
        default: return -1;
    }
    const size_t rb = orc_row_bytes(qtype, n);
    for (int i = 0; i < d; i++) out[i] = dot((const uint8_t *)W + (size_t)i * rb, x, n);
    return 0;
}

/* matmul with the rows split over n_threads pthreads, the way the reference's
 * thread pool splits them (tensor.c:217-236); every row's dot product is the
 * same function, so the output is bit-identical to orc_matmul. */
typedef struct {
    float *out;
    const float *x;
    const uint8_t *W;
    int n, qtype, r0, r1;
    size_t rb;
} mm_task_t;

static void *mm_worker(void *p) {
    mm_task_t *t = (mm_task_t *)p;
    orc_matmul(t->out + t->r0, t->x, t->W + (size_t)t->r0 * t->rb, t->n, t->r1 - t->r0, t->qtype);
    return NULL;
}

int orc_matmul_mt(float *out, const float *x, const void *W, int n, int d, int qtype,
                  int n_threads) {
    if (qtype != ORC_TYPE_Q4_K && qtype != ORC_TYPE_Q6_K && qtype != ORC_TYPE_Q8_0 &&
        qtype != ORC_TYPE_F32)
        return -1; /* the types orc_matmul has a fused dot for */
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    if (n_threads > d) n_threads = d > 0 ? d : 1;
    pthread_t th[64];
    mm_task_t task[64];
    const int per = d / n_threads, extra = d % n_threads;
    int row = 0;
    for (int t = 0; t < n_threads; t++) {
        task[t].out = out;
        task[t].x = x;
        task[t].W = (const uint8_t *)W;
        task[t].n = n;
        task[t].qtype = qtype;
        task[t].rb = orc_row_bytes(qtype, n);
        task[t].r0 = row;
        row += per + (t < extra ? 1 : 0);
        task[t].r1 = row;
    }
    for (int t = 1; t < n_threads; t++) pthread_create(&th[t], NULL, mm_worker, &task[t]);
    mm_worker(&task[0]);
    for (int t = 1; t < n_threads; t++) pthread_join(th[t], NULL);
    return 0;
}
