/*
 * forward_oracle.h -- CPU restatement of picolm's whole forward pass for one
 * token (model.c:746-925, model_forward_ex) and for a prompt
 * (model.c:939-1144, model_forward_prefill), built from the attention and
 * GEMV restatements of attn_oracle.h and quant_oracle.h.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, the smoke entry and the bench's CPU leg
 * load it to check results against; the product never links or calls it.
 *
 * Pinning (tests/test_oracle_forward.py): logits, final residual and every
 * appended KV row bit-exact against the reference's own model_forward and
 * model_forward_prefill (oracle/_ref, driven by ref_harness.c on models
 * assembled from the same host buffers), over LLaMA- and Qwen-shaped models
 * with Q4_K / Q6_K / Q8_0 / F32 matrices, biases and QK-norm; silu against
 * float64 on a grid; the forward on a model whose layers add exact zeros
 * reduces to rmsnorm(embedding) @ output.
 */
#ifndef PICOLM_FORWARD_ORACLE_H
#define PICOLM_FORWARD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One weight matrix: d rows of GGUF blocks (row-major, the reference's
 * in-file layout), qtype a GGUF type id. */
typedef struct {
    int qtype;
    const void *rows;
} orc_matrix;

/* One layer (model.h:40-74 and the run state's dequantized copies,
 * model.c:644-707).  Norm weights and biases are fp32. */
typedef struct {
    const float *attn_norm; /* [n_embd] */
    const float *ffn_norm;  /* [n_embd] */
    orc_matrix q, k, v, o, gate, up, down;
    const float *q_bias;    /* [q_dim]; NULL adds zeros (model.c:781-782) */
    const float *k_bias;    /* [kv_dim] or NULL (model.c:792-795) */
    const float *v_bias;    /* [kv_dim] or NULL (model.c:797-800) */
    const float *o_bias;    /* [n_embd]; NULL adds zeros (model.c:895-896) */
    const float *q_norm;    /* [head_dim] QK-norm weights or NULL */
    const float *k_norm;    /* [head_dim], NULL exactly when q_norm is */
} orc_layer;

typedef struct {
    int n_layers, n_embd, n_ffn, n_heads, n_kv_heads, head_dim, vocab_size,
        max_seq_len, rope_type;
    float rms_norm_eps;
    orc_matrix token_embd;    /* [vocab_size] rows of n_embd */
    const float *output_norm; /* [n_embd] */
    orc_matrix output;        /* [vocab_size] rows of n_embd */
    uint16_t *key_cache;      /* [n_layers][max_seq_len][kv_dim] fp16 bits */
    uint16_t *val_cache;
    const float *rope_cos;    /* [max_seq_len][head_dim/2] */
    const float *rope_sin;
    const orc_layer *layers;  /* [n_layers] */
} orc_model;

/* tensor.c:605-609: x / (1 + expf(-x)) with the host's libm expf. */
float orc_silu(float x);

/* model.c:746-925 for one token at position pos: appends row pos of every
 * layer's caches and writes logits [vocab_size]; x_out (NULL allowed) gets
 * the final normalised residual.  Matmuls split rows over n_threads threads
 * (bit-identical for every count).  0, or -1 for unsupported arguments. */
int orc_forward(const orc_model *m, int token, int pos, float *logits, float *x_out,
                int n_threads);

/* model.c:939-1144: the prompt tokens[0..n_tokens) at positions start_pos..,
 * logits of the last token only (n_tokens >= 1). */
int orc_forward_prefill(const orc_model *m, const int *tokens, int n_tokens, int start_pos,
                        float *logits, float *x_out, int n_threads);

#ifdef __cplusplus
}
#endif

#endif
