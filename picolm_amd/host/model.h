/*
 * model.h -- the part of picolm's model_t that the attention backend reads.
 *
 * Field names and meanings follow the reference (model.h:9 MAX_LAYERS,
 * model.h:22-36 config, model.h:40-84 weights, model.h:88-129 run state;
 * quant.h:49-63 type ids), so gpu_hip.c compiles unchanged against the reference's own model.h
 * when it is dropped into picolm (only these fields are read).  This cut-down
 * copy of the *names* lets the library and its tests build on their own; its
 * binary layout is not picolm's.
 */
#ifndef PICOLM_AMD_MODEL_H
#define PICOLM_AMD_MODEL_H

#include <stdint.h>

#include "quant.h"

#define MAX_LAYERS 64

typedef enum {
    ROPE_TYPE_LLAMA = 0, /* pairs (2i, 2i+1) */
    ROPE_TYPE_QWEN = 1,  /* pairs (i, i + head_dim/2) */
} rope_type_t;

typedef struct {
    int n_embd;
    int n_ffn;
    int n_heads;
    int n_kv_heads;
    int n_layers;
    int vocab_size;
    int max_seq_len;
    int head_dim;
    float rope_freq_base;
    float rms_norm_eps;
    rope_type_t rope_type;
} model_config_t;

typedef struct {
    /* GGUF rows of the projection matrices (host memory, row-major blocks) */
    const void *attn_norm;
    const void *attn_q;
    const void *attn_k;
    const void *attn_v;
    const void *attn_output;
    /* Non-null when the layer has Qwen3's QK-norm; the backend only tests it
     * and reads the dequantized weights from run_state_t. */
    const void *attn_q_norm;
    const void *attn_k_norm;
    const void *ffn_norm;
    const void *ffn_gate;
    const void *ffn_down;
    const void *ffn_up;
    /* biases (Qwen2); NULL when absent */
    const void *attn_q_b;
    const void *attn_k_b;
    const void *attn_v_b;
    const void *attn_output_b;
    gguf_type_t type_attn_q;
    gguf_type_t type_attn_k;
    gguf_type_t type_attn_v;
    gguf_type_t type_attn_output;
    gguf_type_t type_ffn_gate;
    gguf_type_t type_ffn_down;
    gguf_type_t type_ffn_up;
    gguf_type_t type_attn_q_b;
    gguf_type_t type_attn_k_b;
    gguf_type_t type_attn_v_b;
    gguf_type_t type_attn_output_b;
} layer_weights_t;

typedef struct {
    const void *token_embd; /* [vocab_size] GGUF rows of n_embd */
    gguf_type_t type_token_embd;
    const void *output; /* final projection [vocab_size][n_embd] */
    gguf_type_t type_output;
    layer_weights_t layers[MAX_LAYERS];
} model_weights_t;

typedef struct {
    float *x;            /* residual stream [n_embd] */
    float *logits;       /* [vocab_size] */
    uint16_t *key_cache; /* [n_layers][max_seq_len][n_kv_heads*head_dim] fp16 bits */
    uint16_t *val_cache;
    float *rope_cos;     /* [max_seq_len][head_dim/2] */
    float *rope_sin;
    /* dequantized norm weights and biases (model.c:644-707) */
    float *attn_norm_w[MAX_LAYERS];   /* [n_embd] */
    float *ffn_norm_w[MAX_LAYERS];    /* [n_embd] */
    float *attn_q_norm_w[MAX_LAYERS]; /* [head_dim] each (QK-norm layers) */
    float *attn_k_norm_w[MAX_LAYERS];
    float *output_norm_w;             /* [n_embd] */
    float *attn_q_bias[MAX_LAYERS];   /* [n_heads*head_dim], zeros when absent */
    float *attn_k_bias[MAX_LAYERS];   /* [kv_dim] */
    float *attn_v_bias[MAX_LAYERS];   /* [kv_dim] */
    float *attn_output_bias[MAX_LAYERS]; /* [n_embd], zeros when absent */
} run_state_t;

typedef struct {
    model_config_t config;
    model_weights_t weights;
    run_state_t state;
} model_t;

#endif
