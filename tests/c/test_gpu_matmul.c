/*
 * test_gpu_matmul.c -- drives gpu_try_matmul (gpu_hip.c) the way picolm's
 * matmul / matmul_dual call it (tensor.c:200-205, 269-277): gpu_init and
 * gpu_upload_model on a model whose projection matrices are host GGUF rows,
 * then one call per matrix with its own x; a -1 leaves the work to the
 * caller's CPU matmul, which this harness records and skips.
 *
 * Usage: test_gpu_matmul <input.bin> <output.bin>
 * input : int32 [L, n_embd, n_ffn, n_heads, n_kv_heads, head_dim, vocab],
 *         int32 types [L][7] (q, k, v, o, gate, up, down) and type_output,
 *         then for each matrix in that order (layers, then output) its rows
 *         (d * row_bytes) followed by x [n] fp32.
 * output: int32 rc_init, rc_upload, then per matrix int32 rc and float32
 *         out [d]; then int32 rc of three calls that must fall back (an
 *         unknown pointer, a wrong d, a wrong type).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gpu_hip.h"

static size_t row_bytes(int qtype, int n) {
    switch (qtype) {
        case 0: return (size_t)n * 4;
        case 1: return (size_t)n * 2;
        case 8: return (size_t)(n / 32) * 34;
        case 12: return (size_t)(n / 256) * 144;
        case 14: return (size_t)(n / 256) * 210;
        default: return 0;
    }
}

static void *xread(FILE *f, size_t bytes) {
    void *p = malloc(bytes ? bytes : 1);
    if (!p || fread(p, 1, bytes, f) != bytes) {
        fprintf(stderr, "short read\n");
        exit(2);
    }
    return p;
}

typedef struct {
    const void **slot;
    gguf_type_t *type;
    int d, n;
    void *rows;
    float *x;
} mat_t;

int main(int argc, char **argv) {
    if (argc != 3) return 2;
    FILE *fi = fopen(argv[1], "rb");
    if (!fi) return 2;
    int32_t hdr[7];
    if (fread(hdr, 4, 7, fi) != 7) return 2;
    const int L = hdr[0];
    if (L < 1 || L > MAX_LAYERS) return 2;
    int32_t *types = xread(fi, (size_t)(7 * L + 1) * 4);

    model_t m;
    memset(&m, 0, sizeof m);
    model_config_t *c = &m.config;
    c->n_layers = L;
    c->n_embd = hdr[1];
    c->n_ffn = hdr[2];
    c->n_heads = hdr[3];
    c->n_kv_heads = hdr[4];
    c->head_dim = hdr[5];
    c->vocab_size = hdr[6];
    c->max_seq_len = 16;
    c->rope_freq_base = 10000.0f;
    const int kv_dim = c->n_kv_heads * c->head_dim, q_dim = c->n_heads * c->head_dim;
    size_t cache = (size_t)L * c->max_seq_len * kv_dim;
    m.state.key_cache = calloc(cache, 2);
    m.state.val_cache = calloc(cache, 2);
    m.state.rope_cos = calloc((size_t)c->max_seq_len * (c->head_dim / 2), 4);
    m.state.rope_sin = calloc((size_t)c->max_seq_len * (c->head_dim / 2), 4);

    int n_mats = 7 * L + 1;
    mat_t *mats = calloc((size_t)n_mats, sizeof *mats);
    for (int l = 0; l < L; l++) {
        layer_weights_t *lw = &m.weights.layers[l];
        const void **slots[7] = {&lw->attn_q, &lw->attn_k, &lw->attn_v, &lw->attn_output,
                                 &lw->ffn_gate, &lw->ffn_up, &lw->ffn_down};
        gguf_type_t *tys[7] = {&lw->type_attn_q, &lw->type_attn_k, &lw->type_attn_v,
                               &lw->type_attn_output, &lw->type_ffn_gate, &lw->type_ffn_up,
                               &lw->type_ffn_down};
        const int dims[7][2] = {{q_dim, c->n_embd},     {kv_dim, c->n_embd},
                                {kv_dim, c->n_embd},    {c->n_embd, q_dim},
                                {c->n_ffn, c->n_embd},  {c->n_ffn, c->n_embd},
                                {c->n_embd, c->n_ffn}};
        for (int i = 0; i < 7; i++) {
            mat_t *mt = &mats[7 * l + i];
            mt->slot = slots[i];
            mt->type = tys[i];
            mt->d = dims[i][0];
            mt->n = dims[i][1];
            *mt->type = (gguf_type_t)types[7 * l + i];
        }
    }
    mats[7 * L].slot = &m.weights.output;
    mats[7 * L].type = &m.weights.type_output;
    mats[7 * L].d = c->vocab_size;
    mats[7 * L].n = c->n_embd;
    *mats[7 * L].type = (gguf_type_t)types[7 * L];
    for (int i = 0; i < n_mats; i++) {
        mat_t *mt = &mats[i];
        mt->rows = xread(fi, (size_t)mt->d * row_bytes((int)*mt->type, mt->n));
        *mt->slot = mt->rows;
        mt->x = xread(fi, (size_t)mt->n * 4);
    }
    fclose(fi);

    int32_t rc_init = gpu_init(&m);
    int32_t rc_up = rc_init == 0 ? gpu_upload_model(&m) : -1;
    FILE *fo = fopen(argv[2], "wb");
    if (!fo) return 2;
    fwrite(&rc_init, 4, 1, fo);
    fwrite(&rc_up, 4, 1, fo);
    for (int i = 0; i < n_mats; i++) {
        mat_t *mt = &mats[i];
        float *out = calloc((size_t)mt->d, 4);
        int32_t rc = gpu_try_matmul(out, mt->x, mt->rows, mt->n, mt->d, *mt->type);
        fwrite(&rc, 4, 1, fo);
        fwrite(out, 4, (size_t)mt->d, fo);
        free(out);
    }
    /* calls that must fall back: a pointer never uploaded, a wrong d, a wrong
     * type (matrix 0) */
    float *scratch = calloc((size_t)(c->vocab_size + c->n_ffn + c->n_embd), 4);
    int32_t neg[3];
    neg[0] = gpu_try_matmul(scratch, mats[0].x, scratch, mats[0].n, mats[0].d, *mats[0].type);
    neg[1] = gpu_try_matmul(scratch, mats[0].x, mats[0].rows, mats[0].n, mats[0].d - 1,
                            *mats[0].type);
    neg[2] = gpu_try_matmul(scratch, mats[0].x, mats[0].rows, mats[0].n, mats[0].d,
                            (gguf_type_t)(*mats[0].type == GGUF_TYPE_Q8_0 ? GGUF_TYPE_Q4_K
                                                                          : GGUF_TYPE_Q8_0));
    fwrite(neg, 4, 3, fo);
    fclose(fo);
    gpu_shutdown();
    return 0;
}
