/*
 * test_ref_model.c -- the drop-in check of the gpu.h-style boundary with
 * picolm's OWN model_t.
 *
 * Built against the reference's model.h (-I<reference>/picolm), with
 * picolm_amd/host/gpu_hip.c compiled into this program (the way a host
 * program takes it), linked with libpicolm_hip.so (plh_* kernels only) and
 * with oracle/_ref/libpicolm_ref.so: the reference's model.c, tensor.c and
 * quant.c compiled from its sources (test infrastructure).  Every model_t
 * here comes from the reference's allocate_run_state (model.c:560-718)
 * through the harness's ref_model_new / ref_model_new_full, so gpu_init,
 * gpu_upload_model and every hook read picolm's field offsets; the CPU
 * results are the reference's own model_forward_ex / model_forward /
 * model_forward_prefill / matmul / kvcache_save / kvcache_load.
 *
 * Usage:
 *   test_ref_model attn L Hq Hkv D S rope_type n_prompt n_decode n_resume seed out.txt
 *     Attention hooks on the harness's injection model (Wq = Wk = Wv = 0,
 *     q/k/v carried exactly by the biases, Wo = I):
 *       prompt: gpu_try_attention_prefill per layer (start 0, n_prompt rows)
 *               against the reference's decode of the same rows one by one;
 *       decode: gpu_try_attention per layer against model_forward_ex;
 *       persistence (model.c:1146-1259, picolm.c:214-230, 280-283): the GPU
 *               model's host caches are cleared and restored with
 *               gpu_kv_download, saved with kvcache_save and compared byte
 *               for byte with the CPU model's file; a fresh model loads that
 *               file with kvcache_load, gpu_kv_upload pushes it, and n_resume
 *               more tokens are decoded on the device against the CPU run.
 *     A hook that returns -1 is answered as picolm's call sites answer it:
 *     the reference's CPU block runs that layer on the GPU model (counted in
 *     *_fallback).  With the backend lost (PICOLM_HIP_FAIL_AFTER) the host
 *     caches are not cleared and restored, they are the only copy.
 *     Writes one line of key=value results.
 *   test_ref_model forward model.bin out.bin
 *     The whole forward pass: model.bin as tests/c/test_gpu_forward reads it
 *     (GGUF rows, norms, biases, then the step plan).  Model A runs the
 *     reference's model_forward / model_forward_prefill, model B (same
 *     weights) gpu_try_forward / gpu_try_forward_prefill; then every matrix
 *     goes through gpu_try_matmul against the reference's matmul.
 *     out.bin: int32 rc_init, rc_upload; per step int32 rc, float32 GPU
 *     logits [V], GPU x [E], CPU logits [V], CPU x [E]; int32 matmul calls,
 *     matmul bit-exact count; then GPU-model and CPU-model caches
 *     (uint16 key, val each).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gpu_hip.h"
#include "picolm_hip.h"
#include "tensor.h"

/* oracle/_ref/libpicolm_ref.so (oracle/ref_harness.c) */
void *ref_model_new(int n_layers, int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                    float rope_base, int rope_type, int mode, unsigned long long seed,
                    float w_scale);
void *ref_model_new_full(const int *cfg, float rope_base, float eps, const void *const *ptrs,
                         const int *types);
model_t *ref_model(void *h);
void ref_model_free(void *h);
void ref_set_decode_qkv(void *h, int layer, const float *q, const float *k, const float *v);
void ref_decode(void *h, int pos, int n_layers_run, float *attn_out);
void ref_forward(void *h, int token, int pos, float *logits, float *x_out);
void ref_forward_prefill(void *h, const int *tokens, int n_tokens, int start_pos,
                         float *logits, float *x_out);

static uint64_t rng_state;
static double uni(void) {
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return ((double)(z >> 11) + 0.5) * 0x1p-53;
}
static void fill_normal(float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        x[i] = (float)(sqrt(-2.0 * log(uni())) * cos(6.283185307179586 * uni()));
}

/* Attention-output comparison per q head: normwise max|g-r| / max|r| and the
 * elementwise bound |g-r| <= 1e-3 (|r| + rms(r)). */
static void compare(const float *g, const float *r, int n_heads, int D, double *worst,
                    int *elem_bad) {
    for (int h = 0; h < n_heads; h++) {
        double mx = 0, me = 0, ss = 0;
        for (int d = 0; d < D; d++) {
            const double rv = r[h * D + d];
            ss += rv * rv;
            if (fabs(rv) > mx) mx = fabs(rv);
        }
        const double rms = sqrt(ss / D);
        for (int d = 0; d < D; d++) {
            const double e = fabs((double)g[h * D + d] - r[h * D + d]);
            if (e > me) me = e;
            if (!(e <= 1e-3 * (fabs(r[h * D + d]) + rms))) (*elem_bad)++;
        }
        const double nw = mx > 0 ? me / mx : me;
        if (isnan(nw) || isnan(*worst))
            *worst = INFINITY;   /* a NaN anywhere is the worst result */
        else if (nw > *worst)
            *worst = nw;
    }
}

static int caches_equal(const model_t *a, const model_t *b) {
    const model_config_t *c = &a->config;
    const size_t n = (size_t)c->n_layers * c->max_seq_len * c->n_kv_heads * c->head_dim;
    return memcmp(a->state.key_cache, b->state.key_cache, n * 2) == 0 &&
           memcmp(a->state.val_cache, b->state.val_cache, n * 2) == 0;
}

static int files_equal(const char *p1, const char *p2) {
    FILE *a = fopen(p1, "rb"), *b = fopen(p2, "rb");
    int eq = a && b;
    while (eq) {
        const int ca = fgetc(a), cb = fgetc(b);
        if (ca != cb) eq = 0;
        if (ca == EOF || cb == EOF) break;
    }
    if (a) fclose(a);
    if (b) fclose(b);
    return eq;
}

/* One decode token at `pos` on both models: the CPU model runs the
 * reference's model_forward_ex once per layer (layers 0..l, the appends of
 * earlier layers rewrite identical bits), the GPU model calls
 * gpu_try_attention per layer. */
static int decode_both(void *hc, void *hg, model_t *mg, int pos, int L, int q_dim, int kv_dim,
                       float *q, float *k, float *v, float *outc, float *outg,
                       double *worst, int *elem_bad, int *fallback) {
    const model_config_t *c = &mg->config;
    int rc = 0;
    fill_normal(q, (size_t)L * q_dim);
    fill_normal(k, (size_t)L * kv_dim);
    fill_normal(v, (size_t)L * kv_dim);
    for (int l = 0; l < L; l++) {
        ref_set_decode_qkv(hc, l, q + (size_t)l * q_dim, k + (size_t)l * kv_dim,
                           v + (size_t)l * kv_dim);
        ref_set_decode_qkv(hg, l, q + (size_t)l * q_dim, k + (size_t)l * kv_dim,
                           v + (size_t)l * kv_dim);
    }
    for (int l = 0; l < L; l++) {
        ref_decode(hc, pos, l + 1, outc);
        if (gpu_try_attention(mg, l, pos, q + (size_t)l * q_dim, k + (size_t)l * kv_dim,
                              v + (size_t)l * kv_dim, outg) != 0) {
            /* the CPU block of layer l on the GPU model (earlier layers'
             * appends rewrite identical bits) */
            rc = -1;
            ref_decode(hg, pos, l + 1, outg);
            (*fallback)++;
        }
        compare(outg, outc, c->n_heads, c->head_dim, worst, elem_bad);
    }
    return rc;
}

static int run_attn(int argc, char **argv) {
    if (argc != 13) return 2;
    const int L = atoi(argv[2]), Hq = atoi(argv[3]), Hkv = atoi(argv[4]), D = atoi(argv[5]);
    const int S = atoi(argv[6]), rt = atoi(argv[7]), P = atoi(argv[8]), T = atoi(argv[9]);
    const int R = atoi(argv[10]);
    const unsigned long long seed = strtoull(argv[11], NULL, 10);
    const char *out_path = argv[12];
    if (P + T + R > S || L < 1) return 2;
    const float theta = 10000.0f;
    void *hc = ref_model_new(L, Hq, Hkv, D, S, theta, rt, 0, seed, 1.0f);
    void *hg = ref_model_new(L, Hq, Hkv, D, S, theta, rt, 0, seed, 1.0f);
    if (!hc || !hg) return 3;
    model_t *mc = ref_model(hc), *mg = ref_model(hg);
    const int q_dim = Hq * D, kv_dim = Hkv * D, E = mc->config.n_embd;
    rng_state = seed * 7919u + 1u;

    int rc_init = gpu_init(mg);
    int rc_upload = rc_init == 0 ? gpu_upload_model(mg) : -1;

    /* ---- prompt through gpu_try_attention_prefill ---- */
    float *pq = malloc((size_t)L * P * q_dim * 4), *pk = malloc((size_t)L * P * kv_dim * 4);
    float *pv = malloc((size_t)L * P * kv_dim * 4), *pout = malloc((size_t)P * E * 4);
    float *outc = malloc((size_t)E * 4), *outg = malloc((size_t)E * 4);
    fill_normal(pq, (size_t)L * P * q_dim);
    fill_normal(pk, (size_t)L * P * kv_dim);
    fill_normal(pv, (size_t)L * P * kv_dim);
    double prefill_err = 0;
    int prefill_bad = 0, prefill_rc = 0, prefill_fallback = 0;
    for (int l = 0; l < L && P > 0; l++) {
        memset(pout, 0, (size_t)P * E * 4);
        int fell_back = 0;
        if (gpu_try_attention_prefill(mg, l, 0, P, pq + (size_t)l * P * q_dim,
                                      pk + (size_t)l * P * kv_dim, pv + (size_t)l * P * kv_dim,
                                      pout) != 0) {
            prefill_rc = -1;
            fell_back = 1;
            prefill_fallback++;
        }
        /* the reference: the same rows decoded one position at a time (on the
         * GPU model too when the hook fell back) */
        for (int p = 0; p < P; p++) {
            for (int j = 0; j <= l; j++) {
                const float *qj = pq + ((size_t)j * P + p) * q_dim;
                const float *kj = pk + ((size_t)j * P + p) * kv_dim;
                const float *vj = pv + ((size_t)j * P + p) * kv_dim;
                ref_set_decode_qkv(hc, j, qj, kj, vj);
                if (fell_back) ref_set_decode_qkv(hg, j, qj, kj, vj);
            }
            ref_decode(hc, p, l + 1, outc);
            if (fell_back) ref_decode(hg, p, l + 1, pout + (size_t)p * E);
            compare(pout + (size_t)p * E, outc, Hq, D, &prefill_err, &prefill_bad);
        }
    }
    const int prefill_cache_eq = caches_equal(mc, mg);

    /* ---- decode through gpu_try_attention ---- */
    float *q = malloc((size_t)L * q_dim * 4), *k = malloc((size_t)L * kv_dim * 4);
    float *v = malloc((size_t)L * kv_dim * 4);
    double decode_err = 0;
    int decode_bad = 0, decode_rc = 0, decode_fallback = 0;
    for (int t = 0; t < T; t++)
        decode_rc |= decode_both(hc, hg, mg, P + t, L, q_dim, kv_dim, q, k, v, outc, outg,
                                 &decode_err, &decode_bad, &decode_fallback);
    const int decode_cache_eq = caches_equal(mc, mg);

    /* ---- persistence: gpu_kv_download -> kvcache_save, byte-compared ---- */
    const int n_pos = P + T;
    const size_t cache_n = (size_t)L * S * kv_dim;
    int rc_download = -1;
    if (gpu_available()) {
        memset(mg->state.key_cache, 0, cache_n * 2);
        memset(mg->state.val_cache, 0, cache_n * 2);
        rc_download = gpu_kv_download(mg, n_pos);
    }
    const int download_eq = caches_equal(mc, mg);
    char fc[512], fg[512];
    snprintf(fc, sizeof fc, "%s.cpu.kv", out_path);
    snprintf(fg, sizeof fg, "%s.gpu.kv", out_path);
    const int rc_save = kvcache_save(mc, fc, n_pos) | kvcache_save(mg, fg, n_pos);
    const int file_eq = files_equal(fc, fg);
    gpu_shutdown();

    /* ---- a fresh model resumes from the GPU-written file ---- */
    void *hr = ref_model_new(L, Hq, Hkv, D, S, theta, rt, 0, seed, 1.0f);
    model_t *mr = ref_model(hr);
    int rc_reinit = gpu_init(mr);
    int rc_reupload = rc_reinit == 0 ? gpu_upload_model(mr) : -1;
    const int loaded = kvcache_load(mr, fg);
    const int rc_kv_upload = gpu_kv_upload(mr, loaded);
    double resume_err = 0;
    int resume_bad = 0, resume_rc = 0, resume_fallback = 0;
    for (int t = 0; t < R; t++)
        resume_rc |= decode_both(hc, hr, mr, n_pos + t, L, q_dim, kv_dim, q, k, v, outc, outg,
                                 &resume_err, &resume_bad, &resume_fallback);
    const int resume_cache_eq = caches_equal(mc, mr);
    gpu_shutdown();

    FILE *fo = fopen(out_path, "w");
    if (!fo) return 2;
    fprintf(fo,
            "rc_init=%d rc_upload=%d prefill_rc=%d prefill_err=%.6e prefill_bad=%d "
            "prefill_cache_eq=%d decode_rc=%d decode_err=%.6e decode_bad=%d decode_cache_eq=%d "
            "rc_download=%d download_eq=%d rc_save=%d file_eq=%d rc_reinit=%d rc_reupload=%d "
            "loaded=%d rc_kv_upload=%d resume_rc=%d resume_err=%.6e resume_bad=%d "
            "resume_cache_eq=%d prefill_fallback=%d decode_fallback=%d resume_fallback=%d\n",
            rc_init, rc_upload, prefill_rc, prefill_err, prefill_bad, prefill_cache_eq, decode_rc,
            decode_err, decode_bad, decode_cache_eq, rc_download, download_eq, rc_save, file_eq,
            rc_reinit, rc_reupload, loaded, rc_kv_upload, resume_rc, resume_err, resume_bad,
            resume_cache_eq, prefill_fallback, decode_fallback, resume_fallback);
    fclose(fo);
    remove(fc);
    remove(fg);
    ref_model_free(hc);
    ref_model_free(hg);
    ref_model_free(hr);
    return 0;
}

/* ---- forward mode ------------------------------------------------------ */

static size_t row_bytes(int qtype, int n) {
    switch (qtype) {
        case 0: return (size_t)n * 4;
        case 1: return (size_t)n * 2;
        case 2: return (size_t)(n / 32) * 18;
        case 8: return (size_t)(n / 32) * 34;
        case 12: return (size_t)(n / 256) * 144;
        case 14: return (size_t)(n / 256) * 210;
        default: return 0;
    }
}

static void *xread(FILE *f, size_t bytes) {
    void *p = calloc(1, bytes ? bytes : 1);
    if (!p || fread(p, 1, bytes, f) != bytes) {
        fprintf(stderr, "short read\n");
        exit(2);
    }
    return p;
}

enum { SLOTS = 15 };  /* ref_model_new_full's per-layer pointer slots */

static int run_forward(int argc, char **argv) {
    if (argc != 4) return 2;
    FILE *fi = fopen(argv[2], "rb");
    if (!fi) return 2;
    int32_t cfg[9];
    float fl[2];
    if (fread(cfg, 4, 9, fi) != 9 || fread(fl, 4, 2, fi) != 2) return 2;
    const int L = cfg[0], E = cfg[1], F = cfg[2], H = cfg[3], HKV = cfg[4], D = cfg[5];
    const int V = cfg[6], S = cfg[7];
    if (L < 1 || L > MAX_LAYERS) return 2;
    const int Q = H * D, KV = HKV * D;
    int32_t *types = xread(fi, (size_t)(2 + 7 * L) * 4);
    int32_t flags[2];
    if (fread(flags, 4, 2, fi) != 2) return 2;
    const void **ptrs = calloc(3 + (size_t)SLOTS * L, sizeof *ptrs);
    int *ptypes = calloc(3 + (size_t)SLOTS * L, sizeof *ptypes);
    ptypes[0] = types[0];
    ptrs[0] = xread(fi, (size_t)V * row_bytes(types[0], E));
    ptrs[1] = xread(fi, (size_t)E * 4);
    ptypes[2] = types[1];
    ptrs[2] = xread(fi, (size_t)V * row_bytes(types[1], E));
    for (int l = 0; l < L; l++) {
        const void **p = ptrs + 3 + (size_t)SLOTS * l;
        int *t = ptypes + 3 + (size_t)SLOTS * l;
        const int32_t *mt = types + 2 + 7 * l;
        p[0] = xread(fi, (size_t)E * 4);                      /* attn_norm */
        p[7] = xread(fi, (size_t)E * 4);                      /* ffn_norm */
        t[1] = mt[0], p[1] = xread(fi, (size_t)Q * row_bytes(mt[0], E));    /* q */
        t[2] = mt[1], p[2] = xread(fi, (size_t)KV * row_bytes(mt[1], E));   /* k */
        t[3] = mt[2], p[3] = xread(fi, (size_t)KV * row_bytes(mt[2], E));   /* v */
        t[4] = mt[3], p[4] = xread(fi, (size_t)E * row_bytes(mt[3], Q));    /* o */
        t[8] = mt[4], p[8] = xread(fi, (size_t)F * row_bytes(mt[4], E));    /* gate */
        t[10] = mt[5], p[10] = xread(fi, (size_t)F * row_bytes(mt[5], E));  /* up */
        t[9] = mt[6], p[9] = xread(fi, (size_t)E * row_bytes(mt[6], F));    /* down */
        if (flags[0]) {
            p[11] = xread(fi, (size_t)Q * 4);
            p[12] = xread(fi, (size_t)KV * 4);
            p[13] = xread(fi, (size_t)KV * 4);
            p[14] = xread(fi, (size_t)E * 4);
        }
        if (flags[1]) {
            p[5] = xread(fi, (size_t)D * 4);
            p[6] = xread(fi, (size_t)D * 4);
        }
    }
    void *hc = ref_model_new_full(cfg, fl[1], fl[0], ptrs, ptypes);
    void *hg = ref_model_new_full(cfg, fl[1], fl[0], ptrs, ptypes);
    if (!hc || !hg) return 3;
    model_t *mg = ref_model(hg), *mc = ref_model(hc);
    FILE *fo = fopen(argv[3], "wb");
    if (!fo) return 2;
    int32_t rc[2];
    rc[0] = gpu_init(mg);
    rc[1] = rc[0] == 0 ? gpu_upload_model(mg) : -1;
    fwrite(rc, 4, 2, fo);
    float *lc = malloc((size_t)V * 4), *xc = malloc((size_t)E * 4);
    int32_t n_steps;
    if (fread(&n_steps, 4, 1, fi) != 1) return 2;
    for (int s = 0; s < n_steps; s++) {
        int32_t hdr[3];
        if (fread(hdr, 4, 3, fi) != 3) return 2;
        int32_t *toks = xread(fi, (size_t)hdr[2] * 4);
        memset(mg->state.logits, 0, (size_t)V * 4);
        memset(mg->state.x, 0, (size_t)E * 4);
        int32_t r = hdr[0] ? gpu_try_forward_prefill(mg, toks, hdr[2], hdr[1])
                           : gpu_try_forward(mg, toks[0], hdr[1]);
        if (hdr[0])
            ref_forward_prefill(hc, toks, hdr[2], hdr[1], lc, xc);
        else
            ref_forward(hc, toks[0], hdr[1], lc, xc);
        fwrite(&r, 4, 1, fo);
        fwrite(mg->state.logits, 4, (size_t)V, fo);
        fwrite(mg->state.x, 4, (size_t)E, fo);
        fwrite(lc, 4, (size_t)V, fo);
        fwrite(xc, 4, (size_t)E, fo);
        free(toks);
    }
    /* gpu_try_matmul on the reference's own weight pointers and types
     * against its matmul (tensor.c:200-215) */
    int32_t calls = 0, exact = 0;
    float *x = malloc((size_t)(F > E ? F : E) * 4);
    const int maxd = V > F ? (V > E ? V : E) : (F > E ? F : E);
    float *og = malloc((size_t)maxd * 4), *oc = malloc((size_t)maxd * 4);
    for (int l = 0; l < L; l++) {
        const layer_weights_t *lw = &mc->weights.layers[l];
        const struct { const void *w; gguf_type_t t; int n, d; } mats[7] = {
            {lw->attn_q, lw->type_attn_q, E, Q}, {lw->attn_k, lw->type_attn_k, E, KV},
            {lw->attn_v, lw->type_attn_v, E, KV}, {lw->attn_output, lw->type_attn_output, Q, E},
            {lw->ffn_gate, lw->type_ffn_gate, E, F}, {lw->ffn_up, lw->type_ffn_up, E, F},
            {lw->ffn_down, lw->type_ffn_down, F, E}};
        for (int i = 0; i < 7; i++) {
            fill_normal(x, (size_t)mats[i].n);
            if (gpu_try_matmul(og, x, mats[i].w, mats[i].n, mats[i].d, mats[i].t) != 0) continue;
            calls++;
            matmul(oc, x, mats[i].w, mats[i].n, mats[i].d, mats[i].t);
            exact += memcmp(og, oc, (size_t)mats[i].d * 4) == 0;
        }
    }
    fwrite(&calls, 4, 1, fo);
    fwrite(&exact, 4, 1, fo);
    const size_t cache = (size_t)L * S * KV;
    fwrite(mg->state.key_cache, 2, cache, fo);
    fwrite(mg->state.val_cache, 2, cache, fo);
    fwrite(mc->state.key_cache, 2, cache, fo);
    fwrite(mc->state.val_cache, 2, cache, fo);
    gpu_shutdown();
    fclose(fo);
    fclose(fi);
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 2 && strcmp(argv[1], "attn") == 0) return run_attn(argc, argv);
    if (argc >= 2 && strcmp(argv[1], "forward") == 0) return run_forward(argc, argv);
    fprintf(stderr, "usage: test_ref_model attn|forward ...\n");
    return 2;
}
