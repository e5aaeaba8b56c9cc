/*
 * bench_forward.c -- end-to-end latency of gpu_try_forward and
 * gpu_try_forward_prefill (gpu_hip.c) as picolm's model_forward /
 * model_forward_prefill would call them (model.c:742-744, 939): the whole
 * pass on the device, then the logits, x and the appended cache rows back in
 * the host run state, every PCIe transfer and synchronisation included.  The
 * model is a Q4_K_M-style mix (Q4_K token_embd, q, k, o, gate, up; Q6_K v,
 * down, output) of host GGUF rows filled with a fixed byte pattern (finite
 * fp16 scales), unit norms and zero biases: the pass's time does not depend
 * on the values.
 *
 * Usage: bench_forward L n_embd n_ffn n_heads n_kv_heads vocab max_seq pos reps prompt
 * Decode: one untimed token at `pos`, then `reps` timed tokens at pos+1...
 * Prefill: one untimed `prompt`-token prefill at position 0, then `reps`
 * timed ones.  KV: gpu_kv_download then gpu_kv_upload of every layer's rows
 * 0..pos+reps-1 (one untimed pair, then `reps` timed).  Prints one JSON line
 * of medians and means in microseconds.
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

/* rows of d GGUF rows of n values of type qtype, filled with 0x21 */
static void *fill_rows(int qtype, int d, int n) {
    const size_t bytes = (size_t)d * row_bytes(qtype, n);
    void *p = malloc(bytes);
    if (p) memset(p, 0x21, bytes);
    return p;
}

static float *fill_f32(int n, float v) {
    float *p = malloc((size_t)n * sizeof(float));
    if (p)
        for (int i = 0; i < n; i++) p[i] = v;
    return p;
}

static void summary(const char *tag, double *t, int reps) {
    double mean = 0.0;
    for (int r = 0; r < reps; r++) mean += t[r] / reps;
    qsort(t, (size_t)reps, sizeof(double), cmp_d);
    printf("\"%s_us_median\": %.1f, \"%s_us_mean\": %.1f", tag, t[reps / 2], tag, mean);
}

int main(int argc, char **argv) {
    if (argc != 11) {
        fprintf(stderr,
                "usage: bench_forward L n_embd n_ffn n_heads n_kv_heads vocab max_seq pos reps "
                "prompt\n");
        return 2;
    }
    const int L = atoi(argv[1]), E = atoi(argv[2]), F = atoi(argv[3]), Hq = atoi(argv[4]);
    const int Hkv = atoi(argv[5]), V = atoi(argv[6]), S = atoi(argv[7]), pos = atoi(argv[8]);
    const int reps = atoi(argv[9]), prompt = atoi(argv[10]);
    if (L < 1 || L > MAX_LAYERS || reps < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || E % Hq ||
        E % 256 || F % 256 || V < 1 || S < 2 || pos < 0 || pos + reps >= S || prompt < 1 ||
        prompt > S)
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
    c->max_seq_len = S;
    c->rope_freq_base = 10000.0f;
    c->rms_norm_eps = 1e-5f;
    run_state_t *st = &m.state;
    const size_t cache = (size_t)L * S * kv_dim;
    st->key_cache = calloc(cache, 2);
    st->val_cache = calloc(cache, 2);
    st->rope_cos = fill_f32(S * (D / 2), 1.0f);
    st->rope_sin = fill_f32(S * (D / 2), 0.0f);
    st->x = fill_f32(E, 0.0f);
    st->logits = fill_f32(V, 0.0f);
    st->output_norm_w = fill_f32(E, 1.0f);
    if (!st->key_cache || !st->val_cache || !st->rope_cos || !st->rope_sin || !st->x ||
        !st->logits || !st->output_norm_w)
        return 3;

    model_weights_t *w = &m.weights;
    w->type_token_embd = GGUF_TYPE_Q4_K;
    w->token_embd = fill_rows(GGUF_TYPE_Q4_K, V, E);
    w->type_output = GGUF_TYPE_Q6_K;
    w->output = fill_rows(GGUF_TYPE_Q6_K, V, E);
    if (!w->token_embd || !w->output) return 3;
    for (int l = 0; l < L; l++) {
        layer_weights_t *lw = &w->layers[l];
        const void **slots[7] = {&lw->attn_q, &lw->attn_k, &lw->attn_v, &lw->attn_output,
                                 &lw->ffn_gate, &lw->ffn_up, &lw->ffn_down};
        gguf_type_t *tys[7] = {&lw->type_attn_q, &lw->type_attn_k, &lw->type_attn_v,
                               &lw->type_attn_output, &lw->type_ffn_gate, &lw->type_ffn_up,
                               &lw->type_ffn_down};
        const int dims[7][2] = {{E, E}, {kv_dim, E}, {kv_dim, E}, {E, E},
                                {F, E}, {F, E},      {E, F}};
        for (int j = 0; j < 7; j++) {
            const int qt = (j == 2 || j == 6) ? GGUF_TYPE_Q6_K : GGUF_TYPE_Q4_K;
            *tys[j] = (gguf_type_t)qt;
            *slots[j] = fill_rows(qt, dims[j][0], dims[j][1]);
            if (!*slots[j]) return 3;
        }
        st->attn_norm_w[l] = fill_f32(E, 1.0f);
        st->ffn_norm_w[l] = fill_f32(E, 1.0f);
        st->attn_q_bias[l] = fill_f32(E, 0.0f);
        st->attn_output_bias[l] = fill_f32(E, 0.0f);
        if (!st->attn_norm_w[l] || !st->ffn_norm_w[l] || !st->attn_q_bias[l] ||
            !st->attn_output_bias[l])
            return 3;
    }

    if (gpu_init(&m) != 0 || gpu_upload_model(&m) != 0) {
        fprintf(stderr, "gpu_init / gpu_upload_model failed\n");
        return 4;
    }
    int *tokens = malloc((size_t)prompt * sizeof(int));
    double *dec = malloc((size_t)reps * sizeof(double));
    double *pre = malloc((size_t)reps * sizeof(double));
    if (!tokens || !dec || !pre) return 3;
    for (int i = 0; i < prompt; i++) tokens[i] = (i * 7919) % V;
    for (int r = -1; r < reps; r++) {
        const double t0 = now_us();
        if (gpu_try_forward(&m, (r + 2) % V, pos + 1 + r) != 0) {
            fprintf(stderr, "gpu_try_forward fell back at position %d\n", pos + 1 + r);
            return 5;
        }
        if (r >= 0) dec[r] = now_us() - t0;
    }
    for (int r = -1; r < reps; r++) {
        const double t0 = now_us();
        if (gpu_try_forward_prefill(&m, tokens, prompt, 0) != 0) {
            fprintf(stderr, "gpu_try_forward_prefill fell back\n");
            return 5;
        }
        if (r >= 0) pre[r] = now_us() - t0;
    }
    /* kvcache_save / kvcache_load coherence (model.c:1146-1259): every layer's
     * rows 0..kv_pos-1 down into the host caches and back up */
    const int kv_pos = pos + reps;
    double *kvd = malloc((size_t)reps * sizeof(double));
    double *kvu = malloc((size_t)reps * sizeof(double));
    if (!kvd || !kvu) return 1;
    for (int r = -1; r < reps; r++) {
        double t0 = now_us();
        if (gpu_kv_download(&m, kv_pos) != 0) {
            fprintf(stderr, "gpu_kv_download failed\n");
            return 1;
        }
        double t1 = now_us();
        if (gpu_kv_upload(&m, kv_pos) != 0) {
            fprintf(stderr, "gpu_kv_upload failed\n");
            return 1;
        }
        double t2 = now_us();
        if (r >= 0) {
            kvd[r] = t1 - t0;
            kvu[r] = t2 - t1;
        }
    }
    printf("{\"hook\": \"gpu_try_forward\", \"pos\": %d, \"prompt\": %d, \"reps\": %d, ", pos + 1,
           prompt, reps);
    summary("decode", dec, reps);
    printf(", ");
    summary("prefill", pre, reps);
    printf(", \"kv_pos\": %d, ", kv_pos);
    summary("kv_download", kvd, reps);
    printf(", ");
    summary("kv_upload", kvu, reps);
    printf("}\n");
    gpu_shutdown();
    return 0;
}
