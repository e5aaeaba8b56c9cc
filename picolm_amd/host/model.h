/*
 * model.h -- the part of picolm's model_t that the attention backend reads.
 *
 * Field names and meanings follow the reference (model.h:15-36 config,
 * model.h:98-106 run state), so gpu_hip.c compiles unchanged against the
 * reference's own model.h when it is dropped into picolm (only these fields
 * are read).  This cut-down copy of the *names* lets the library and its
 * tests build on their own; its binary layout is not picolm's.
 */
#ifndef PICOLM_AMD_MODEL_H
#define PICOLM_AMD_MODEL_H

#include <stdint.h>

typedef enum {
    ROPE_TYPE_LLAMA = 0, /* pairs (2i, 2i+1) */
    ROPE_TYPE_QWEN = 1,  /* pairs (i, i + head_dim/2) */
} rope_type_t;

typedef struct {
    int n_embd;
    int n_heads;
    int n_kv_heads;
    int n_layers;
    int max_seq_len;
    int head_dim;
    float rope_freq_base;
    rope_type_t rope_type;
} model_config_t;

typedef struct {
    uint16_t *key_cache; /* [n_layers][max_seq_len][n_kv_heads*head_dim] fp16 bits */
    uint16_t *val_cache;
    float *rope_cos;     /* [max_seq_len][head_dim/2] */
    float *rope_sin;
} run_state_t;

typedef struct {
    model_config_t config;
    run_state_t state;
} model_t;

#endif
