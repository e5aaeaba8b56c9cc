/*
 * bench_boundary.c -- end-to-end latency of the gpu.h-style attention hooks
 * (gpu_hip.c) as picolm's forward passes would see it: host q/k/v in, host
 * output and host cache rows back, every PCIe copy and synchronisation
 * included (the device-resident figures of the kernels alone are the bench's
 * other numbers).
 *
 * Usage: bench_boundary L Hq Hkv D S theta pos n_prompt reps
 *   n_prompt = 0: one decode token at position pos, the L per-layer
 *                 gpu_try_attention calls of model_forward_ex (model.c:819);
 *   n_prompt > 0: a prompt of n_prompt tokens at positions pos.., the L
 *                 per-layer gpu_try_attention_prefill calls of
 *                 model_forward_prefill (model.c:1039).
 * Rows 0..pos-1 of the host caches hold seeded N(0,1) values in fp16 before
 * gpu_upload_model copies them to the device.  One untimed token (or
 * prompt) first, then `reps` timed ones.  Prints one JSON line:
 * per-call and per-token microseconds (median and mean over reps).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "gpu_hip.h"
#include "picolm_hip.h"

static uint64_t rs = 0x243F6A8885A308D3ull;
static float nrand(void) {
    uint64_t a = (rs += 0x9E3779B97F4A7C15ull), b = (rs += 0x9E3779B97F4A7C15ull);
    a = (a ^ (a >> 31)) * 0xBF58476D1CE4E5B9ull;
    b = (b ^ (b >> 29)) * 0x94D049BB133111EBull;
    const double u1 = ((double)(a >> 11) + 0.5) * 0x1p-53, u2 = (double)(b >> 11) * 0x1p-53;
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

static uint16_t f16_bits(float f) {  /* truncating conversion: only cache contents */
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint32_t sgn = (u >> 16) & 0x8000u;
    const int e = (int)((u >> 23) & 0xFFu) - 127 + 15;
    if (e <= 0) return (uint16_t)sgn;
    if (e >= 31) return (uint16_t)(sgn | 0x7C00u);
    return (uint16_t)(sgn | ((uint32_t)e << 10) | ((u & 0x7FFFFFu) >> 13));
}

static double now_us(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e6 + ts.tv_nsec * 1e-3;
}

static int cmp_d(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

int main(int argc, char **argv) {
    if (argc != 10) {
        fprintf(stderr, "usage: bench_boundary L Hq Hkv D S theta pos n_prompt reps\n");
        return 2;
    }
    const int L = atoi(argv[1]), Hq = atoi(argv[2]), Hkv = atoi(argv[3]), D = atoi(argv[4]);
    const int S = atoi(argv[5]), pos = atoi(argv[7]), P = atoi(argv[8]), reps = atoi(argv[9]);
    const float theta = (float)atof(argv[6]);
    if (L < 1 || L > MAX_LAYERS || reps < 1 || pos < 0 || pos + (P > 0 ? P : 1) > S) return 2;
    const size_t q_dim = (size_t)Hq * D, kv_dim = (size_t)Hkv * D;
    const int n_tok = P > 0 ? P : 1;

    model_t m;
    memset(&m, 0, sizeof m);
    m.config.n_embd = (int)q_dim;
    m.config.n_heads = Hq;
    m.config.n_kv_heads = Hkv;
    m.config.n_layers = L;
    m.config.max_seq_len = S;
    m.config.head_dim = D;
    m.config.rope_freq_base = theta;
    m.config.rms_norm_eps = 1e-5f;
    m.config.rope_type = ROPE_TYPE_LLAMA;
    const size_t cache = (size_t)L * S * kv_dim;
    m.state.key_cache = calloc(cache, 2);
    m.state.val_cache = calloc(cache, 2);
    m.state.rope_cos = malloc((size_t)S * (D / 2) * 4);
    m.state.rope_sin = malloc((size_t)S * (D / 2) * 4);
    if (!m.state.key_cache || !m.state.val_cache || !m.state.rope_cos || !m.state.rope_sin)
        return 3;
    plh_rope_tables_host(m.state.rope_cos, m.state.rope_sin, S, D, theta);
    for (int l = 0; l < L; l++)
        for (size_t i = 0; i < (size_t)pos * kv_dim; i++) {
            const size_t at = (size_t)l * S * kv_dim + i;
            m.state.key_cache[at] = f16_bits(nrand());
            m.state.val_cache[at] = f16_bits(nrand());
        }
    float *q = malloc((size_t)L * n_tok * q_dim * 4), *k = malloc((size_t)L * n_tok * kv_dim * 4);
    float *v = malloc((size_t)L * n_tok * kv_dim * 4), *out = malloc((size_t)n_tok * q_dim * 4);
    for (size_t i = 0; i < (size_t)L * n_tok * q_dim; i++) q[i] = nrand();
    for (size_t i = 0; i < (size_t)L * n_tok * kv_dim; i++) k[i] = nrand(), v[i] = nrand();

    if (gpu_init(&m) != 0 || gpu_upload_model(&m) != 0) {
        fprintf(stderr, "gpu_init / gpu_upload_model failed\n");
        return 4;
    }
    double *tok = malloc((size_t)reps * sizeof(double));
    int bad = 0;
    for (int r = -1; r < reps; r++) {
        const double t0 = now_us();
        for (int l = 0; l < L; l++) {
            const size_t qo = (size_t)l * n_tok * q_dim, ko = (size_t)l * n_tok * kv_dim;
            const int rc = P > 0 ? gpu_try_attention_prefill(&m, l, pos, P, q + qo, k + ko, v + ko,
                                                             out)
                                 : gpu_try_attention(&m, l, pos, q + qo, k + ko, v + ko, out);
            bad |= rc != 0;
        }
        if (r >= 0) tok[r] = now_us() - t0;
    }
    gpu_shutdown();
    if (bad) {
        fprintf(stderr, "a hook returned -1\n");
        return 5;
    }
    double mean = 0;
    for (int r = 0; r < reps; r++) mean += tok[r] / reps;
    qsort(tok, (size_t)reps, sizeof(double), cmp_d);
    const double med = tok[reps / 2];
    printf("{\"hook\": \"%s\", \"calls_per_token\": %d, \"us_per_token_median\": %.2f, "
           "\"us_per_token_mean\": %.2f, \"us_per_call_median\": %.2f, \"reps\": %d}\n",
           P > 0 ? "gpu_try_attention_prefill" : "gpu_try_attention", L, med, mean, med / L,
           reps);
    return 0;
}
