/*
 * picolm_hip.h -- device-level C ABI of libpicolm_hip.so (gfx950 / MI355X).
 *
 * Plain pointers and sizes only.  Every pointer named "device" is HBM memory
 * obtained from plh_malloc (or any hipMalloc allocation on the current
 * device).  All work is queued on the library's single stream; calls return
 * once the work is queued unless stated otherwise.
 *
 * Return convention (gpu.h:23-26 of the reference): 0 = done, -1 = not
 * handled / failed; plh_last_error() then holds a message.
 *
 * KV-cache layout (model.h:98-100, model.c:802-805, bit-exact with the
 * reference): uint16 fp16 bit patterns,
 *     cache[((layer * max_seq_len + t) * n_kv_heads + kv_head) * head_dim + d]
 * with key_cache and val_cache as two such blocks.  RoPE tables are
 * [max_seq_len][head_dim/2] fp32, cos and sin (model.c:545-556).
 */
#ifndef PICOLM_HIP_H
#define PICOLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PLH_ROPE_LLAMA 0 /* pairs (2i, 2i+1), model.h:15-18 */
#define PLH_ROPE_QWEN 1  /* pairs (i, i + head_dim/2)        */

/* ---- lifecycle (the device half of gpu_init / gpu_shutdown, gpu.h:12-29) -- */
int plh_init(int device);
void plh_shutdown(void);
int plh_available(void);
const char *plh_last_error(void);
int plh_device_count(void);

/* ---- device memory and synchronisation ---------------------------------- */
void *plh_malloc(size_t bytes);
int plh_free(void *dptr);
int plh_memcpy_htod(void *dst, const void *src, size_t bytes);
int plh_memcpy_dtoh(void *dst, const void *src, size_t bytes);
int plh_memcpy_dtod(void *dst, const void *src, size_t bytes);
int plh_memset(void *dst, int value, size_t bytes);
int plh_synchronize(void);

/* ---- timing on the library stream (hipEvents) -------------------------- */
void *plh_event_create(void);
int plh_event_record(void *ev);
float plh_event_elapsed_ms(void *start, void *stop); /* waits for stop */
void plh_event_destroy(void *ev);

/* ---- HIP graphs of the library stream ------------------------------------ */
/* Everything queued between begin and end (decode launches, event records) is
 * captured instead of run; plh_graph_launch replays it.  Decode launches need
 * no memset and allocate nothing once the workspace has been sized by one
 * eager call of the same shape, so they can be captured. */
int plh_capture_begin(void);
void *plh_capture_end(void); /* instantiated graph, or NULL */
int plh_graph_launch(void *graph);
void plh_graph_destroy(void *graph);

/* ---- host-side RoPE tables ---------------------------------------------- */
/* Replaces model.c:545-556 (init_rope_tables) with the same libm calls in the
 * same order, so the tables are bit-identical to the reference's on the same
 * host.  cos_tab/sin_tab are HOST arrays [max_seq_len][head_dim/2]. */
void plh_rope_tables_host(float *cos_tab, float *sin_tab, int max_seq_len,
                          int head_dim, float freq_base);

/* ---- fp16 conversion (quant.c:41-78 semantics) --------------------------- */
/* dst[i] = fp32_to_fp16(src[i]) with round-half-away-from-zero, on device. */
int plh_f32_to_f16(const float *src, uint16_t *dst, size_t n);
/* Order-independent checksum of the conversion over the fp32 bit patterns
 * [first, first+count): sum of (f16(x)+1) * (mix64(x)|1) mod 2^64.  Blocking;
 * result written to *checksum (host).  Used to sweep all 2^32 inputs. */
int plh_f16_checksum(uint64_t first, uint64_t count, uint64_t *checksum);

/* ---- decode attention ---------------------------------------------------- */
/* Replaces model.c:819-892 (rope, FP16 append, online-softmax GQA attention)
 * for one token at position `pos`, for `n_launch_layers` consecutive layers
 * starting at `layer0` in ONE launch (n_launch_layers = 1 is the per-layer
 * call of model_forward_ex; more layers is the bench's all-layers step, not a
 * reference call).  Per launched layer li (all device pointers):
 *   q   + li*n_heads*head_dim     fp32 q (not rotated; left unmodified)
 *   k,v + li*n_kv_heads*head_dim  fp32 k (not rotated), v
 *   out + li*n_heads*head_dim     fp32 attention output
 * The kernel rotates q and k with table row `pos`, writes f16(k_rot), f16(v)
 * into row `pos` of layer layer0+li of the caches, and attends over rows
 * 0..pos.  Supported: head_dim 64 or 128, n_heads % n_kv_heads == 0,
 * |q| < 65504. */
int plh_attn_decode(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                    int max_seq_len, int rope_type, int layer0,
                    int n_launch_layers, int pos, const float *q,
                    const float *k, const float *v, uint16_t *key_cache,
                    uint16_t *val_cache, const float *rope_cos,
                    const float *rope_sin, float *out);

/* ---- prefill attention -------------------------------------------------- */
/* Replaces model.c:1039-1089 (per prompt token: rope, FP16 append, online-
 * softmax GQA attention) for n_tokens tokens at positions start_pos.. and
 * n_launch_layers consecutive layers from layer0 (1 = the per-layer call of
 * model_forward_prefill).  Per launched layer li (device pointers):
 *   q   + li*n_tokens*n_heads*head_dim     [n_tokens][n_heads*head_dim] fp32
 *   k,v + li*n_tokens*n_kv_heads*head_dim  [n_tokens][kv_dim] fp32
 *   out + li*n_tokens*out_stride            row bi at out + bi*out_stride
 * Rows start_pos..start_pos+n_tokens-1 of each layer's caches are written
 * (f16 of rotated k, f16 of v, reference rounding); token bi attends over
 * rows 0..start_pos+bi, the prefix rows coming from the cache as the
 * reference's kvcache_load leaves them.  out_stride is a multiple of 4 and at
 * least n_heads*head_dim (the reference uses n_embd).  n_tokens = 0 is a
 * no-op. */
int plh_attn_prefill(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                     int max_seq_len, int rope_type, int layer0,
                     int n_launch_layers, int start_pos, int n_tokens,
                     const float *q, const float *k, const float *v,
                     uint16_t *key_cache, uint16_t *val_cache,
                     const float *rope_cos, const float *rope_sin, float *out,
                     int out_stride);

/* ---- Qwen3 QK-norm variants ----------------------------------------------- */
/* The two calls above with the QK-norm of model.c:807-817 (decode) and
 * 1029-1037 (prefill) in front of the rotation: every q head row is
 * RMS-normalised with q_norm and every k head row with k_norm, epsilon
 * norm_eps (the model's rms_norm_eps), as the reference's rmsnorm
 * (tensor.c:425-492) computes it in its x86-64 AVX2 build -- the cached k
 * rows stay bit-exact.  q_norm, k_norm: device pointers, [n_launch_layers]
 * [head_dim] fp32 (layer li of the launch at + li*head_dim); both null gives
 * the plain call, one null is an error. */
int plh_attn_decode_qknorm(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                           int max_seq_len, int rope_type, int layer0,
                           int n_launch_layers, int pos, const float *q,
                           const float *k, const float *v, uint16_t *key_cache,
                           uint16_t *val_cache, const float *rope_cos,
                           const float *rope_sin, float *out, const float *q_norm,
                           const float *k_norm, float norm_eps);
int plh_attn_prefill_qknorm(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                            int max_seq_len, int rope_type, int layer0,
                            int n_launch_layers, int start_pos, int n_tokens,
                            const float *q, const float *k, const float *v,
                            uint16_t *key_cache, uint16_t *val_cache,
                            const float *rope_cos, const float *rope_sin, float *out,
                            int out_stride, const float *q_norm, const float *k_norm,
                            float norm_eps);

/* ---- weight GEMV (gpu_try_matmul's path) --------------------------------- */
/* Replaces the reference's matmul row loop (tensor.c:200-215) for GGUF types
 * Q4_K (12), Q6_K (14) and Q8_0 (8) -- the types its Vulkan backend offloads
 * (gpu.c:595-602): out[i] = vec_dot(row i of W, x), bit-identical to the
 * reference's fused dequantize + dot products in its x86-64 (AVX2 + FMA)
 * build (quant.c:390-452, 517-582, 627-659).  W is a d x n matrix, n a
 * multiple of the block (256, 256, 32).
 *
 * plh_gemv_packed_bytes: size of the device copy (0: type or shape has no
 * kernel).  plh_gemv_upload: packs the reference's row-major blocks (HOST
 * pointer, d * row_bytes) into that device buffer (synchronous).
 * plh_gemv_pack_host: the same packing into a HOST buffer (no device use),
 * for callers that stage uploads themselves.
 * plh_gemv: x [n] and out [d] fp32 device pointers, W the packed copy;
 * queued on the library stream. */
size_t plh_gemv_packed_bytes(int qtype, int n, int d);
int plh_gemv_upload(int qtype, int n, int d, const void *host_rows, void *dev);
int plh_gemv_pack_host(int qtype, int n, int d, const void *host_rows, void *host_packed);
int plh_gemv(int qtype, int n, int d, const void *dev, const float *x, float *out);

/* Tuning knobs (bench sweeps).  key 1: decode target workgroups per launch
 * (0 = default); key 2: decode contexts of at most this many positions are
 * not split (multiple of 128, 0 = default); key 3: GEMV rows per thread
 * (1, 2, 4, 8; 0 = default). */
int plh_set_tuning(int key, int value);

#ifdef __cplusplus
}
#endif

#endif /* PICOLM_HIP_H */
