/*
 * test_gpu_forward.c -- drives gpu_try_forward / gpu_try_forward_prefill
 * (gpu_hip.c) the way picolm's model_forward / model_forward_prefill would
 * call them (model.c:742-744, 939): a model_t assembled from host buffers
 * (GGUF rows for the matrices, the run state's dequantized norms and biases),
 * gpu_init + gpu_upload_model, then a plan of prefill and decode steps.
 *
 * Usage: test_gpu_forward <input.bin> <output.bin>
 * input : int32 cfg[9] = {L, n_embd, n_ffn, n_heads, n_kv_heads, head_dim,
 *         vocab, max_seq_len, rope_type}, float32 {eps, rope_base},
 *         int32 types[2 + 7L] = {embd, output, then per layer q, k, v, o,
 *         gate, up, down}, int32 {has_bias, has_qkn}; then token_embd rows,
 *         output_norm [E], output rows; per layer attn_norm [E], ffn_norm [E],
 *         the seven matrices' rows in that order, then (has_bias) q_bias [Q],
 *         k_bias [KV], v_bias [KV], o_bias [E], then (has_qkn) q_norm [D],
 *         k_norm [D].  Then int32 n_steps and per step {kind (0 decode,
 *         1 prefill), start_pos, n_tokens, tokens[n_tokens]}.
 * output: int32 rc_init, rc_upload; per step int32 rc, float32 logits [V],
 *         float32 x [E]; then the host caches key, val (uint16 each
 *         [L][S][KV]).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gpu_hip.h"
#include "picolm_hip.h"

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

int main(int argc, char **argv) {
    if (argc != 3) return 2;
    FILE *fi = fopen(argv[1], "rb");
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

    model_t m;
    memset(&m, 0, sizeof m);
    model_config_t *c = &m.config;
    c->n_layers = L, c->n_embd = E, c->n_ffn = F, c->n_heads = H, c->n_kv_heads = HKV;
    c->head_dim = D, c->vocab_size = V, c->max_seq_len = S;
    c->rope_type = (rope_type_t)cfg[8];
    c->rms_norm_eps = fl[0];
    c->rope_freq_base = fl[1];
    model_weights_t *w = &m.weights;
    run_state_t *st = &m.state;
    w->type_token_embd = (gguf_type_t)types[0];
    w->token_embd = xread(fi, (size_t)V * row_bytes(types[0], E));
    st->output_norm_w = xread(fi, (size_t)E * 4);
    w->type_output = (gguf_type_t)types[1];
    w->output = xread(fi, (size_t)V * row_bytes(types[1], E));
    static float zeros_q[65536], zeros_e[65536];
    for (int l = 0; l < L; l++) {
        layer_weights_t *lw = &w->layers[l];
        const int32_t *t = types + 2 + 7 * l;
        st->attn_norm_w[l] = xread(fi, (size_t)E * 4);
        st->ffn_norm_w[l] = xread(fi, (size_t)E * 4);
        lw->attn_norm = st->attn_norm_w[l];
        lw->ffn_norm = st->ffn_norm_w[l];
        lw->type_attn_q = (gguf_type_t)t[0];
        lw->attn_q = xread(fi, (size_t)Q * row_bytes(t[0], E));
        lw->type_attn_k = (gguf_type_t)t[1];
        lw->attn_k = xread(fi, (size_t)KV * row_bytes(t[1], E));
        lw->type_attn_v = (gguf_type_t)t[2];
        lw->attn_v = xread(fi, (size_t)KV * row_bytes(t[2], E));
        lw->type_attn_output = (gguf_type_t)t[3];
        lw->attn_output = xread(fi, (size_t)E * row_bytes(t[3], Q));
        lw->type_ffn_gate = (gguf_type_t)t[4];
        lw->ffn_gate = xread(fi, (size_t)F * row_bytes(t[4], E));
        lw->type_ffn_up = (gguf_type_t)t[5];
        lw->ffn_up = xread(fi, (size_t)F * row_bytes(t[5], E));
        lw->type_ffn_down = (gguf_type_t)t[6];
        lw->ffn_down = xread(fi, (size_t)E * row_bytes(t[6], F));
        /* no bias: the run state's zero buffers (model.c:678-707) */
        st->attn_q_bias[l] = zeros_q;
        st->attn_output_bias[l] = zeros_e;
        if (flags[0]) {
            st->attn_q_bias[l] = xread(fi, (size_t)Q * 4);
            st->attn_k_bias[l] = xread(fi, (size_t)KV * 4);
            st->attn_v_bias[l] = xread(fi, (size_t)KV * 4);
            st->attn_output_bias[l] = xread(fi, (size_t)E * 4);
            lw->attn_q_b = st->attn_q_bias[l];
            lw->attn_k_b = st->attn_k_bias[l];
            lw->attn_v_b = st->attn_v_bias[l];
            lw->attn_output_b = st->attn_output_bias[l];
        }
        if (flags[1]) {
            st->attn_q_norm_w[l] = xread(fi, (size_t)D * 4);
            st->attn_k_norm_w[l] = xread(fi, (size_t)D * 4);
            lw->attn_q_norm = st->attn_q_norm_w[l];
            lw->attn_k_norm = st->attn_k_norm_w[l];
        }
    }
    const size_t cache = (size_t)L * S * KV;
    st->key_cache = calloc(cache, 2);
    st->val_cache = calloc(cache, 2);
    st->rope_cos = calloc((size_t)S * (D / 2), 4);
    st->rope_sin = calloc((size_t)S * (D / 2), 4);
    st->logits = calloc((size_t)V, 4);
    st->x = calloc((size_t)E, 4);
    plh_rope_tables_host(st->rope_cos, st->rope_sin, S, D, c->rope_freq_base);

    FILE *fo = fopen(argv[2], "wb");
    if (!fo) return 2;
    int32_t rc[2];
    rc[0] = gpu_init(&m);
    rc[1] = rc[0] == 0 ? gpu_upload_model(&m) : -1;
    fwrite(rc, 4, 2, fo);
    int32_t n_steps;
    if (fread(&n_steps, 4, 1, fi) != 1) return 2;
    for (int sidx = 0; sidx < n_steps; sidx++) {
        int32_t hdr[3];
        if (fread(hdr, 4, 3, fi) != 3) return 2;
        int32_t *toks = xread(fi, (size_t)hdr[2] * 4);
        memset(st->logits, 0, (size_t)V * 4);
        memset(st->x, 0, (size_t)E * 4);
        int32_t r = hdr[0] ? gpu_try_forward_prefill(&m, toks, hdr[2], hdr[1])
                           : gpu_try_forward(&m, toks[0], hdr[1]);
        fwrite(&r, 4, 1, fo);
        fwrite(st->logits, 4, (size_t)V, fo);
        fwrite(st->x, 4, (size_t)E, fo);
        free(toks);
    }
    fwrite(st->key_cache, 2, cache, fo);
    fwrite(st->val_cache, 2, cache, fo);
    gpu_shutdown();
    fclose(fo);
    fclose(fi);
    return 0;
}
