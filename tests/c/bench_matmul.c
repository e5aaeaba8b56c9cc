/*
 * bench_matmul.c -- end-to-end latency of gpu_try_matmul (gpu_hip.c) as
 * picolm's matmul / matmul_dual call it (tensor.c:200-205, 269-277): one call
 * per projection of every layer (q, k, v, o, gate, up, down), then the output
 * projection, each with host x in and host out back, every PCIe transfer and
 * synchronisation included.  The weights are host GGUF rows of a Q4_K_M-style
 * mix (Q4_K q, k, o, gate, up; Q6_K v, down, output) filled with a fixed byte
 * pattern (finite fp16 scales): the GEMV's time does not depend on the values.
 *
 * Usage: bench_matmul L n_embd n_ffn n_heads n_kv_heads vocab reps
 * One untimed token first, then `reps` timed ones.  Prints one JSON line:
 * per-call (median over the calls of all timed tokens) and per-token
 * microseconds (median and mean over reps).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "gpu_hip.h"

static size_t row_bytes(int qtype, int n) {
    return qtype == GGUF_TYPE_Q4_K ? (size_t)(n / 256) * 144 : (size_t)(n / 256) * 210;
}

static double now_us(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec * 1e6 + t.tv_nsec / 1e3;
}

static int cmp_d(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

typedef struct {
    const void *rows;
    gguf_type_t type;
    int d, n;
} mat_t;

int main(int argc, char **argv) {
    if (argc != 8) {
        fprintf(stderr, "usage: bench_matmul L n_embd n_ffn n_heads n_kv_heads vocab reps\n");
        return 2;
    }
    const int L = atoi(argv[1]), E = atoi(argv[2]), F = atoi(argv[3]), Hq = atoi(argv[4]);
    const int Hkv = atoi(argv[5]), V = atoi(argv[6]), reps = atoi(argv[7]);
    if (L < 1 || L > MAX_LAYERS || reps < 1 || Hq < 1 || Hkv < 1 || E % Hq || E % 256 ||
        F % 256 || V < 1)
        return 2;
    const int D = E / Hq, kv_dim = Hkv * D;

    model_t m;
    memset(&m, 0, sizeof m);
    model_config_t *c = &m.config;
    c->n_layers = L;
    c->n_embd = E;
    c->n_ffn = F;
    c->n_heads = Hq;
    c->n_kv_heads = Hkv;
    c->head_dim = D;
    c->vocab_size = V;
    c->max_seq_len = 16;
    c->rope_freq_base = 10000.0f;
    c->rms_norm_eps = 1e-5f;
    const size_t cache = (size_t)L * c->max_seq_len * kv_dim;
    m.state.key_cache = calloc(cache, 2);
    m.state.val_cache = calloc(cache, 2);
    m.state.rope_cos = calloc((size_t)c->max_seq_len * (D / 2), 4);
    m.state.rope_sin = calloc((size_t)c->max_seq_len * (D / 2), 4);
    if (!m.state.key_cache || !m.state.val_cache || !m.state.rope_cos || !m.state.rope_sin)
        return 3;

    const int n_mats = 7 * L + 1;
    mat_t *mats = calloc((size_t)n_mats, sizeof *mats);
    int max_n = 0, max_d = 0;
    for (int i = 0; i < n_mats; i++) {
        const int l = i / 7, j = i % 7;
        mat_t *mt = &mats[i];
        if (i == 7 * L) {
            mt->type = GGUF_TYPE_Q6_K, mt->d = V, mt->n = E;
        } else {
            const int dims[7][2] = {{E, E}, {kv_dim, E}, {kv_dim, E}, {E, E},
                                    {F, E}, {F, E},      {E, F}};
            const int q6 = j == 2 || j == 6;
            mt->type = q6 ? GGUF_TYPE_Q6_K : GGUF_TYPE_Q4_K;
            mt->d = dims[j][0], mt->n = dims[j][1];
        }
        const size_t bytes = (size_t)mt->d * row_bytes((int)mt->type, mt->n);
        unsigned char *rows = malloc(bytes);
        if (!rows) return 3;
        memset(rows, 0x21, bytes);  /* fp16 scales 0x2121: finite, small */
        mt->rows = rows;
        if (i < 7 * L) {
            layer_weights_t *lw = &m.weights.layers[l];
            const void **slots[7] = {&lw->attn_q, &lw->attn_k, &lw->attn_v, &lw->attn_output,
                                     &lw->ffn_gate, &lw->ffn_up, &lw->ffn_down};
            gguf_type_t *tys[7] = {&lw->type_attn_q, &lw->type_attn_k, &lw->type_attn_v,
                                   &lw->type_attn_output, &lw->type_ffn_gate,
                                   &lw->type_ffn_up, &lw->type_ffn_down};
            *slots[j] = rows;
            *tys[j] = mt->type;
        } else {
            m.weights.output = rows;
            m.weights.type_output = mt->type;
        }
        if (mt->n > max_n) max_n = mt->n;
        if (mt->d > max_d) max_d = mt->d;
    }
    float *x = malloc((size_t)max_n * 4), *out = malloc((size_t)max_d * 4);
    if (!x || !out) return 3;
    for (int i = 0; i < max_n; i++) x[i] = (float)((i * 37) % 101) / 101.0f - 0.5f;

    if (gpu_init(&m) != 0 || gpu_upload_model(&m) != 0) {
        fprintf(stderr, "gpu_init / gpu_upload_model failed\n");
        return 4;
    }
    double *per_tok = malloc((size_t)reps * sizeof(double));
    double *per_call = malloc((size_t)reps * n_mats * sizeof(double));
    for (int r = -1; r < reps; r++) {
        const double t0 = now_us();
        for (int i = 0; i < n_mats; i++) {
            const double c0 = now_us();
            if (gpu_try_matmul(out, x, mats[i].rows, mats[i].n, mats[i].d, mats[i].type) != 0) {
                fprintf(stderr, "gpu_try_matmul fell back on matrix %d\n", i);
                return 5;
            }
            if (r >= 0) per_call[(size_t)r * n_mats + i] = now_us() - c0;
        }
        if (r >= 0) per_tok[r] = now_us() - t0;
    }
    double mean = 0.0;
    for (int r = 0; r < reps; r++) mean += per_tok[r] / reps;
    qsort(per_tok, (size_t)reps, sizeof(double), cmp_d);
    qsort(per_call, (size_t)reps * n_mats, sizeof(double), cmp_d);
    printf("{\"hook\": \"gpu_try_matmul\", \"calls_per_token\": %d, \"us_per_token_median\": %.2f, "
           "\"us_per_token_mean\": %.2f, \"us_per_call_median\": %.2f, \"reps\": %d}\n",
           n_mats, per_tok[reps / 2], mean, per_call[(size_t)reps * n_mats / 2], reps);
    gpu_shutdown();
    return 0;
}
