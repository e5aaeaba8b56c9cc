/*
 * gpu_hip.h -- picolm's GPU backend interface (gpu.h) for the MI355X
 * attention block.
 *
 * Same conventions as the reference's gpu.h (gpu.h:7-42): one global backend,
 * lifecycle gpu_init -> gpu_upload_model -> ... -> gpu_shutdown, and every
 * gpu_try_* returns 0 when it did the work or -1 when the caller must run its
 * own CPU code (nothing half-applied).  Without USE_HIP the calls are inline
 * stubs returning -1 / 0, as gpu.h:31-42 does without USE_VULKAN.
 *
 * Environment (gpu.c:143-150, 241-252 style):
 *   PICOLM_HIP_DISABLE=1  gpu_init fails, everything stays on the CPU
 *   PICOLM_HIP_DEVICE=N   device index (default 0)
 *   PICOLM_GPU_LAYERS=N   only layers < N use the GPU; later layers get -1
 *   PICOLM_HIP_MATMUL=0   upload no weight matrices (gpu_try_matmul -> -1)
 *   PICOLM_HIP_FORWARD=0  no whole-forward offload (gpu_try_forward* -> -1)
 *
 * Host caches stay authoritative: every successful call copies the rows it
 * appended back into m->state.key_cache / val_cache, so the CPU fallback and
 * kvcache_save (model.c:1158-1197) see bit-identical data.
 */
#ifndef PICOLM_GPU_HIP_H
#define PICOLM_GPU_HIP_H

#include "model.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifdef USE_HIP

/* gpu.h:12-15 -- select the device, create the stream.  0 or -1. */
int gpu_init(const model_t *m);
/* gpu.h:17-20 -- allocate the device FP16 KV cache [L][S][kv_dim] and RoPE
 * tables, upload the host tables and cache, and (unless PICOLM_HIP_MATMUL=0)
 * the Q4_K / Q6_K / Q8_0 projection matrices of layers < PICOLM_GPU_LAYERS
 * and the output matrix (gpu.c:427-464), packed for the GEMV.  0 or -1. */
int gpu_upload_model(const model_t *m);
/* gpu.h:22 -- 1 when initialised and uploaded. */
int gpu_available(void);
/* gpu.h:24-26 -- out[d] = W[d,n] @ x[n] on the device for an uploaded
 * matrix (found by its host pointer W), bit-identical to the reference's
 * CPU matmul (x86-64 AVX2 build).  -1 when W was not uploaded, its type has
 * no kernel, or n / d / qtype differ from the upload: the caller's CPU
 * matmul runs (tensor.c:202-205). */
int gpu_try_matmul(float *out, const float *x, const void *W, int n, int d,
                   gguf_type_t qtype);
/* gpu.h:28 -- drain and release everything. */
void gpu_shutdown(void);

/* Replaces model.c:819-892 for layer `layer` at position `pos`: RoPE of q/k,
 * FP16 append of row pos, online-softmax GQA attention over rows 0..pos.
 * q [n_heads*head_dim], k and v [n_kv_heads*head_dim] are read (not rotated
 * in place; nothing reads them afterwards), out [n_heads*head_dim] written. */
int gpu_try_attention(model_t *m, int layer, int pos, float *q, float *k,
                      const float *v, float *out);
/* Replaces model.c:1039-1089 for n_tokens prompt rows at start_pos..:
 * q [n_tokens][n_heads*head_dim], k/v [n_tokens][kv_dim]; out row bi at
 * out + bi*n_embd (model.c:1057). */
int gpu_try_attention_prefill(model_t *m, int layer, int start_pos, int n_tokens,
                              float *q, float *k, const float *v, float *out);
/* Replaces model_forward_ex(m, token, pos, n_layers) (model.c:746-925) with
 * the whole forward pass on the device: fills m->state.logits and m->state.x
 * (the final normalised residual) and appends row pos of every layer's
 * caches (device and host).  Available when gpu_upload_model put every
 * layer's seven projections and the output matrix on the device (GEMV
 * types), the embedding type is F32/F16/Q4_0/Q8_0/Q4_K/Q6_K and the q /
 * output biases are F32 in the file; -1 otherwise (nothing changed).  The
 * logits match the reference's to the attention/silu exp tolerance; the
 * first layer's KV rows bit for bit. */
int gpu_try_forward(model_t *m, int token, int pos);
/* Replaces model_forward_prefill(m, tokens, n_tokens, start_pos)
 * (model.c:939-1144): logits / x of the last token, rows start_pos.. of
 * every layer appended. */
int gpu_try_forward_prefill(model_t *m, const int *tokens, int n_tokens, int start_pos);
/* KV coherence for kvcache_save / kvcache_load (model.c:1146-1259): copy rows
 * 0..n_pos-1 of every layer the device handles (layers < PICOLM_GPU_LAYERS)
 * device -> host (download) or host -> device (upload); the other layers'
 * rows live in the host cache only and are left alone.  0 or -1. */
int gpu_kv_download(const model_t *m, int n_pos);
int gpu_kv_upload(const model_t *m, int n_pos);

#else /* !USE_HIP */

static inline int gpu_init(const model_t *m) { (void)m; return -1; }
static inline int gpu_upload_model(const model_t *m) { (void)m; return -1; }
static inline int gpu_available(void) { return 0; }
static inline int gpu_try_matmul(float *o, const float *x, const void *W, int n, int d,
                                 gguf_type_t qt) {
    (void)o; (void)x; (void)W; (void)n; (void)d; (void)qt; return -1;
}
static inline void gpu_shutdown(void) {}
static inline int gpu_try_attention(model_t *m, int l, int p, float *q, float *k,
                                    const float *v, float *o) {
    (void)m; (void)l; (void)p; (void)q; (void)k; (void)v; (void)o; return -1;
}
static inline int gpu_try_attention_prefill(model_t *m, int l, int s, int n, float *q,
                                            float *k, const float *v, float *o) {
    (void)m; (void)l; (void)s; (void)n; (void)q; (void)k; (void)v; (void)o; return -1;
}
static inline int gpu_try_forward(model_t *m, int t, int p) {
    (void)m; (void)t; (void)p; return -1;
}
static inline int gpu_try_forward_prefill(model_t *m, const int *t, int n, int s) {
    (void)m; (void)t; (void)n; (void)s; return -1;
}
static inline int gpu_kv_download(const model_t *m, int n) { (void)m; (void)n; return -1; }
static inline int gpu_kv_upload(const model_t *m, int n) { (void)m; (void)n; return -1; }

#endif /* USE_HIP */

#ifdef __cplusplus
}
#endif

#endif /* PICOLM_GPU_HIP_H */
