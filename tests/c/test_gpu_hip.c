/*
 * test_gpu_hip.c -- drives the gpu.h-style boundary (gpu_hip.c) the way
 * picolm's forward passes would: per layer, gpu_try_attention_prefill at the
 * point of model.c:1039 for the prompt, then gpu_try_attention at the point
 * of model.c:819 for each generated token; a call returning -1 leaves the
 * work to the caller's CPU block, which this harness records and skips.
 *
 * Usage: test_gpu_hip <input.bin> <output.bin>
 * input : int32 [L, Hq, Hkv, D, S, rope_type, n_prompt, n_decode, qkn_mask],
 *         float32 theta, rms_norm_eps, then prompt q [L][P][q_dim],
 *         k, v [L][P][kv_dim], then decode q [T][L][q_dim], k, v [T][L][kv_dim],
 *         then QK-norm weights q_norm [L][D], k_norm [L][D]; bit l of qkn_mask
 *         gives layer l a non-null attn_q_norm (Qwen3, model.c:807)
 * output: int32 [rc_init, rc_upload, rc_download_roundtrip, rc_upload_roundtrip],
 *         int32 rc_prefill[L], int32 rc_decode[T][L],
 *         float32 prefill out [L][P][n_embd], decode out [T][L][q_dim],
 *         uint16 host key cache, val cache.  Layers whose calls returned -1
 *         hold a stand-in for the CPU block's rows in rows 0..P+T-1:
 *         key 0x3C00 | ((l + 3r + i) & 0xFF), val 0x4000 | ((l + 5r + i) & 0xFF)
 *         for element i of row r of layer l.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gpu_hip.h"
#include "picolm_hip.h"

static void *xread(FILE *f, size_t bytes) {
    void *p = malloc(bytes ? bytes : 1);
    if (!p || fread(p, 1, bytes, f) != bytes) {
        fprintf(stderr, "short read\n");
        exit(2);
    }
    return p;
}

int main(int argc, char **argv) {
    if (argc != 3) return 2;
    FILE *fi = fopen(argv[1], "rb");
    if (!fi) return 2;
    int32_t hdr[9];
    float theta, eps;
    if (fread(hdr, 4, 9, fi) != 9 || fread(&theta, 4, 1, fi) != 1 || fread(&eps, 4, 1, fi) != 1)
        return 2;
    const int L = hdr[0], Hq = hdr[1], Hkv = hdr[2], D = hdr[3], S = hdr[4], rt = hdr[5];
    const int P = hdr[6], T = hdr[7], qkn_mask = hdr[8];
    if (L < 1 || L > 31) return 2;
    const size_t q_dim = (size_t)Hq * D, kv_dim = (size_t)Hkv * D;
    float *pq = xread(fi, (size_t)L * P * q_dim * 4);
    float *pk = xread(fi, (size_t)L * P * kv_dim * 4);
    float *pv = xread(fi, (size_t)L * P * kv_dim * 4);
    float *dq = xread(fi, (size_t)T * L * q_dim * 4);
    float *dk = xread(fi, (size_t)T * L * kv_dim * 4);
    float *dv = xread(fi, (size_t)T * L * kv_dim * 4);
    float *qn = xread(fi, (size_t)L * D * 4);
    float *kn = xread(fi, (size_t)L * D * 4);
    fclose(fi);

    model_t m;
    memset(&m, 0, sizeof m);
    m.config.n_embd = (int)q_dim;
    m.config.n_heads = Hq;
    m.config.n_kv_heads = Hkv;
    m.config.n_layers = L;
    m.config.max_seq_len = S;
    m.config.head_dim = D;
    m.config.rope_freq_base = theta;
    m.config.rms_norm_eps = eps;
    m.config.rope_type = (rope_type_t)rt;
    for (int l = 0; l < L; l++) {
        /* the backend tests the weight pointer and reads the dequantized rows */
        m.weights.layers[l].attn_q_norm = ((qkn_mask >> l) & 1) ? (const void *)qn : NULL;
        m.weights.layers[l].attn_k_norm = m.weights.layers[l].attn_q_norm;
        m.state.attn_q_norm_w[l] = qn + (size_t)l * D;
        m.state.attn_k_norm_w[l] = kn + (size_t)l * D;
    }
    size_t cache_elems = (size_t)L * S * kv_dim;
    m.state.key_cache = calloc(cache_elems, 2); /* zero-filled like model.c:612-619 */
    m.state.val_cache = calloc(cache_elems, 2);
    m.state.rope_cos = malloc((size_t)S * (D / 2) * 4);
    m.state.rope_sin = malloc((size_t)S * (D / 2) * 4);
    plh_rope_tables_host(m.state.rope_cos, m.state.rope_sin, S, D, theta);

    int32_t rc[4] = {0, 0, 0, 0};
    int32_t *rc_pre = calloc((size_t)L, 4);
    int32_t *rc_dec = calloc((size_t)T * L, 4);
    float *out_pre = calloc((size_t)L * P * q_dim, 4);
    float *out_dec = calloc((size_t)T * L * q_dim, 4);

    rc[0] = gpu_init(&m);
    rc[1] = rc[0] == 0 ? gpu_upload_model(&m) : -1;

    /* prompt: model_forward_prefill's layer loop, attention block per layer */
    for (int l = 0; l < L; l++) {
        rc_pre[l] = gpu_try_attention_prefill(&m, l, 0, P, pq + (size_t)l * P * q_dim,
                                              pk + (size_t)l * P * kv_dim,
                                              pv + (size_t)l * P * kv_dim,
                                              out_pre + (size_t)l * P * q_dim);
    }
    /* generation: model_forward_ex's layer loop at pos P + t */
    for (int t = 0; t < T; t++)
        for (int l = 0; l < L; l++) {
            size_t i = (size_t)t * L + l;
            rc_dec[i] = gpu_try_attention(&m, l, P + t, dq + i * q_dim, dk + i * kv_dim,
                                          dv + i * kv_dim, out_dec + i * q_dim);
        }

    /* Layers whose calls fell back: the caller's CPU block appends their
     * rows to the host cache only.  Stand-in rows (a fixed pattern) take
     * that place here; the device never sees them, and downloads must
     * leave them as they are. */
    int n_pos = P + T;
    unsigned char *dev_layer = calloc((size_t)L, 1);
    for (int l = 0; l < L; l++) {
        int ok = P == 0 || rc_pre[l] == 0;
        for (int t = 0; t < T; t++) ok = ok && rc_dec[(size_t)t * L + l] == 0;
        dev_layer[l] = (unsigned char)ok;
        if (ok || !gpu_available()) continue;
        for (int r = 0; r < n_pos; r++)
            for (size_t i = 0; i < kv_dim; i++) {
                size_t at = ((size_t)l * S + r) * kv_dim + i;
                m.state.key_cache[at] = (uint16_t)(0x3C00u | ((l + 3u * r + i) & 0xFFu));
                m.state.val_cache[at] = (uint16_t)(0x4000u | ((l + 5u * r + i) & 0xFFu));
            }
    }
    /* kvcache_save / kvcache_load coherence: download into cleared host rows
     * of the device's layers must give back the same bytes and leave the
     * CPU layers' rows alone; upload then download too */
    const size_t layer_elems = (size_t)S * kv_dim;
    uint16_t *kcopy = malloc(cache_elems * 2), *vcopy = malloc(cache_elems * 2);
    memcpy(kcopy, m.state.key_cache, cache_elems * 2);
    memcpy(vcopy, m.state.val_cache, cache_elems * 2);
    if (gpu_available()) {
        for (int l = 0; l < L; l++)
            if (dev_layer[l]) {
                memset(m.state.key_cache + (size_t)l * layer_elems, 0, layer_elems * 2);
                memset(m.state.val_cache + (size_t)l * layer_elems, 0, layer_elems * 2);
            }
        rc[2] = gpu_kv_download(&m, n_pos);
        if (rc[2] == 0 && (memcmp(kcopy, m.state.key_cache, cache_elems * 2) ||
                           memcmp(vcopy, m.state.val_cache, cache_elems * 2)))
            rc[2] = 1;
        rc[3] = gpu_kv_upload(&m, n_pos);
        if (rc[3] == 0) {
            for (int l = 0; l < L; l++)
                if (dev_layer[l]) {
                    memset(m.state.key_cache + (size_t)l * layer_elems, 0, layer_elems * 2);
                    memset(m.state.val_cache + (size_t)l * layer_elems, 0, layer_elems * 2);
                }
            rc[3] = gpu_kv_download(&m, n_pos);
            if (rc[3] == 0 && (memcmp(kcopy, m.state.key_cache, cache_elems * 2) ||
                               memcmp(vcopy, m.state.val_cache, cache_elems * 2)))
                rc[3] = 1;
        }
    } else {
        rc[2] = gpu_kv_download(&m, n_pos);
        rc[3] = gpu_kv_upload(&m, n_pos);
    }
    gpu_shutdown();

    FILE *fo = fopen(argv[2], "wb");
    if (!fo) return 2;
    fwrite(rc, 4, 4, fo);
    fwrite(rc_pre, 4, (size_t)L, fo);
    fwrite(rc_dec, 4, (size_t)T * L, fo);
    fwrite(out_pre, 4, (size_t)L * P * q_dim, fo);
    fwrite(out_dec, 4, (size_t)T * L * q_dim, fo);
    fwrite(kcopy, 2, cache_elems, fo);
    fwrite(vcopy, 2, cache_elems, fo);
    fclose(fo);
    return 0;
}
