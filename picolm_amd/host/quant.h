/*
 * quant.h -- the GGUF type ids of picolm's quant.h (quant.h:49-63), the only
 * part of it the attention/GEMV backend needs.  Names and values follow the
 * reference so gpu_hip.c compiles unchanged against either header.
 */
#ifndef PICOLM_AMD_QUANT_H
#define PICOLM_AMD_QUANT_H

typedef enum {
    GGUF_TYPE_F32 = 0,
    GGUF_TYPE_F16 = 1,
    GGUF_TYPE_Q4_0 = 2,
    GGUF_TYPE_Q4_1 = 3,
    GGUF_TYPE_Q5_0 = 6,
    GGUF_TYPE_Q5_1 = 7,
    GGUF_TYPE_Q8_0 = 8,
    GGUF_TYPE_Q8_1 = 9,
    GGUF_TYPE_Q2_K = 10,
    GGUF_TYPE_Q3_K = 11,
    GGUF_TYPE_Q4_K = 12,
    GGUF_TYPE_Q5_K = 13,
    GGUF_TYPE_Q6_K = 14,
} gguf_type_t;

#endif
