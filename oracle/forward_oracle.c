/*
 * forward_oracle.c -- restatement of picolm's forward pass (test oracle; see
 * forward_oracle.h for what it follows and how it is pinned).
 *
 * Every step calls the pinned restatements: orc_dequantize_row for the
 * embedding (quant.c:265-276), orc_rmsnorm (tensor.c:425-492),
 * orc_matmul_mt for the projections (tensor.c:200-254; the reference's
 * matmul_dual / matmul_batch compute the same vec_dot per row and token),
 * orc_attn_decode_qkn for QK-norm + RoPE + FP16 append + attention
 * (model.c:807-892).  The element-wise steps are written out here:
 * vec_add (tensor.c:635-657) a[i] + b[i], silu (tensor.c:605-609),
 * elemwise_mul (tensor.c:611-633) a[i] * b[i].  Built with
 * -ffp-contract=off, like the reference's -std=c11 build.
 */
#include "forward_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "attn_oracle.h"
#include "quant_oracle.h"

float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* Matrices of the types with a fused dot product (quant.c:713-718); the
 * reference's dequantize-then-dot fallback for other types is not restated. */
static int matrix_ok(orc_matrix w, int n) {
    return w.rows != NULL && orc_row_bytes(w.qtype, n) > 0 &&
           (w.qtype == ORC_TYPE_Q4_K || w.qtype == ORC_TYPE_Q6_K || w.qtype == ORC_TYPE_Q8_0 ||
            w.qtype == ORC_TYPE_F32);
}

static int model_ok(const orc_model *m) {
    if (!m || m->n_layers < 1 || m->n_embd < 1 || m->n_ffn < 1 || m->n_heads < 1 ||
        m->n_kv_heads < 1 || m->vocab_size < 1 || m->max_seq_len < 1 || !m->layers)
        return 0;
    if (m->head_dim < 2 || m->head_dim > 256 || (m->head_dim & 1) ||
        m->n_heads % m->n_kv_heads)
        return 0;
    const int q_dim = m->n_heads * m->head_dim;
    if (!m->output_norm || !m->key_cache || !m->val_cache || !m->rope_cos || !m->rope_sin)
        return 0;
    if (!m->token_embd.rows || orc_row_bytes(m->token_embd.qtype, m->n_embd) == 0)
        return 0;
    if (!matrix_ok(m->output, m->n_embd)) return 0;
    for (int l = 0; l < m->n_layers; l++) {
        const orc_layer *lw = &m->layers[l];
        if (!lw->attn_norm || !lw->ffn_norm) return 0;
        if (!matrix_ok(lw->q, m->n_embd) || !matrix_ok(lw->k, m->n_embd) ||
            !matrix_ok(lw->v, m->n_embd) || !matrix_ok(lw->o, q_dim) ||
            !matrix_ok(lw->gate, m->n_embd) || !matrix_ok(lw->up, m->n_embd) ||
            !matrix_ok(lw->down, m->n_ffn))
            return 0;
        if ((lw->q_norm == NULL) != (lw->k_norm == NULL)) return 0;
    }
    return 1;
}

typedef struct {
    float *x, *xb, *xb2, *q, *k, *v, *hb, *hb2;
} acts;

static int acts_new(const orc_model *m, acts *a) {
    const size_t q_dim = (size_t)m->n_heads * m->head_dim;
    const size_t kv_dim = (size_t)m->n_kv_heads * m->head_dim;
    const size_t wide = q_dim > (size_t)m->n_embd ? q_dim : (size_t)m->n_embd;
    const size_t total = 3 * wide + q_dim + 2 * kv_dim + 2 * (size_t)m->n_ffn;
    float *p = (float *)calloc(total, sizeof(float));
    if (!p) return -1;
    a->x = p; p += wide;
    a->xb = p; p += wide;
    a->xb2 = p; p += wide;
    a->q = p; p += q_dim;
    a->k = p; p += kv_dim;
    a->v = p; p += kv_dim;
    a->hb = p; p += m->n_ffn;
    a->hb2 = p;
    return 0;
}

static void add_into(float *a, const float *b, int n) {
    for (int i = 0; i < n; i++) a[i] = a[i] + b[i];
}

static void add_zeros(float *a, int n) {
    for (int i = 0; i < n; i++) a[i] = a[i] + 0.0f;
}

/* One token through every layer: a->x holds the embedding on entry and the
 * residual stream on exit.  bias_always selects model_forward_ex's bias
 * handling (q and output biases always added, zeros when absent,
 * model.c:781-782 / 895-896) over model_forward_prefill's (only present
 * biases, model.c:1002-1017 / 1095-1099). */
static int layers_one_token(const orc_model *m, acts *a, int pos, int bias_always,
                            int n_threads) {
    const int dim = m->n_embd, n_ffn = m->n_ffn;
    const int q_dim = m->n_heads * m->head_dim, kv_dim = m->n_kv_heads * m->head_dim;
    for (int l = 0; l < m->n_layers; l++) {
        const orc_layer *lw = &m->layers[l];
        orc_rmsnorm(a->xb, a->x, lw->attn_norm, dim, m->rms_norm_eps);
        orc_matmul_mt(a->q, a->xb, lw->q.rows, dim, q_dim, lw->q.qtype, n_threads);
        orc_matmul_mt(a->k, a->xb, lw->k.rows, dim, kv_dim, lw->k.qtype, n_threads);
        orc_matmul_mt(a->v, a->xb, lw->v.rows, dim, kv_dim, lw->v.qtype, n_threads);
        if (lw->q_bias)
            add_into(a->q, lw->q_bias, q_dim);
        else if (bias_always)
            add_zeros(a->q, q_dim);
        if (lw->k_bias) add_into(a->k, lw->k_bias, kv_dim);
        if (lw->v_bias) add_into(a->v, lw->v_bias, kv_dim);
        if (orc_attn_decode_qkn(m->n_layers, m->n_heads, m->n_kv_heads, m->head_dim,
                                m->max_seq_len, m->rope_type, l, pos, a->q, a->k, a->v,
                                m->key_cache, m->val_cache, m->rope_cos, m->rope_sin, a->xb,
                                lw->q_norm, lw->k_norm, m->rms_norm_eps) != 0)
            return -1;
        orc_matmul_mt(a->xb2, a->xb, lw->o.rows, q_dim, dim, lw->o.qtype, n_threads);
        if (lw->o_bias)
            add_into(a->xb2, lw->o_bias, dim);
        else if (bias_always)
            add_zeros(a->xb2, dim);
        add_into(a->x, a->xb2, dim);

        orc_rmsnorm(a->xb, a->x, lw->ffn_norm, dim, m->rms_norm_eps);
        orc_matmul_mt(a->hb, a->xb, lw->gate.rows, dim, n_ffn, lw->gate.qtype, n_threads);
        orc_matmul_mt(a->hb2, a->xb, lw->up.rows, dim, n_ffn, lw->up.qtype, n_threads);
        for (int i = 0; i < n_ffn; i++) a->hb[i] = orc_silu(a->hb[i]);
        for (int i = 0; i < n_ffn; i++) a->hb[i] = a->hb[i] * a->hb2[i];
        orc_matmul_mt(a->xb, a->hb, lw->down.rows, n_ffn, dim, lw->down.qtype, n_threads);
        add_into(a->x, a->xb, dim);
    }
    return 0;
}

static void embed(const orc_model *m, int token, float *x) {
    const size_t rb = orc_row_bytes(m->token_embd.qtype, m->n_embd);
    orc_dequantize_row(m->token_embd.qtype,
                       (const uint8_t *)m->token_embd.rows + (size_t)token * rb, x, m->n_embd);
}

static void head(const orc_model *m, acts *a, float *logits, float *x_out, int n_threads) {
    orc_rmsnorm(a->xb, a->x, m->output_norm, m->n_embd, m->rms_norm_eps);
    orc_matmul_mt(logits, a->xb, m->output.rows, m->n_embd, m->vocab_size, m->output.qtype,
                  n_threads);
    if (x_out) memcpy(x_out, a->xb, (size_t)m->n_embd * sizeof(float));
}

int orc_forward(const orc_model *m, int token, int pos, float *logits, float *x_out,
                int n_threads) {
    if (!model_ok(m) || !logits || token < 0 || token >= m->vocab_size || pos < 0 ||
        pos >= m->max_seq_len)
        return -1;
    acts a;
    if (acts_new(m, &a) != 0) return -1;
    embed(m, token, a.x);
    int rc = layers_one_token(m, &a, pos, 1, n_threads);
    if (rc == 0) head(m, &a, logits, x_out, n_threads);
    free(a.x);
    return rc;
}

/* Token-major order gives the reference's layer-major prefill bit for bit:
 * token bi at layer l reads rows 0..start_pos+bi of layer l, all written
 * before it in either order, and every other step is per token. */
int orc_forward_prefill(const orc_model *m, const int *tokens, int n_tokens, int start_pos,
                        float *logits, float *x_out, int n_threads) {
    if (!model_ok(m) || !logits || !tokens || n_tokens < 1 || start_pos < 0 ||
        (long)start_pos + n_tokens > (long)m->max_seq_len)
        return -1;
    for (int bi = 0; bi < n_tokens; bi++)
        if (tokens[bi] < 0 || tokens[bi] >= m->vocab_size) return -1;
    acts a;
    if (acts_new(m, &a) != 0) return -1;
    int rc = 0;
    for (int bi = 0; bi < n_tokens && rc == 0; bi++) {
        embed(m, tokens[bi], a.x);
        rc = layers_one_token(m, &a, start_pos + bi, 0, n_threads);
    }
    if (rc == 0) head(m, &a, logits, x_out, n_threads);
    free(a.x);
    return rc;
}
