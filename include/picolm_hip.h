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
/* height rows of width bytes, row i from src + i*spitch to dst + i*dpitch
 * (blocking): the per-layer rows of one position in one call. */
int plh_memcpy2d_dtoh(void *dst, size_t dpitch, const void *src, size_t spitch,
                      size_t width, size_t height);
/* plh_memcpy2d_dtoh in the other direction (host rows to device rows),
 * blocking: every layer's rows of a cache in one call. */
int plh_memcpy2d_htod(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width,
                      size_t height);
int plh_memset(void *dst, int value, size_t bytes);
int plh_synchronize(void);
/* Pinned (page-locked) host memory, for staging copies that the DMA engines
 * run without an intermediate bounce: plh_host_alloc returns NULL on
 * failure. */
void *plh_host_alloc(size_t bytes);
int plh_host_free(void *host);
/* Copies queued on the library stream without waiting (the host side should
 * be pinned memory from plh_host_alloc and must stay untouched until a later
 * plh_synchronize). */
int plh_memcpy_htod_async(void *dst, const void *src, size_t bytes);
int plh_memcpy_dtoh_async(void *dst, const void *src, size_t bytes);
/* plh_memcpy2d_dtoh queued the same way, without waiting. */
int plh_memcpy2d_dtoh_async(void *dst, size_t dpitch, const void *src, size_t spitch,
                            size_t width, size_t height);
/* Up to four strided copies as ONE kernel launch on the library stream,
 * without waiting: copy i moves `height` rows of `width` bytes from `src`
 * (rows `spitch` bytes apart) to `dst` (rows `dpitch` apart).  Either side
 * may be device memory or pinned host memory from plh_host_alloc (the kernel
 * reads and writes it over PCIe), so a host collecting several results after
 * a pass pays one launch rather than one DMA command per copy.  Copies must
 * not overlap each other; rows of a copy must not overlap (pitch >= width).
 * Returns -1 (plh_last_error) for n outside 1..4, a null pointer with a
 * non-empty copy, or a pitch below the width; empty copies are skipped. */
typedef struct {
    void *dst;
    size_t dpitch;
    const void *src;
    size_t spitch;
    size_t width, height;
} plh_copy2d;
int plh_copy2d_batch_async(const plh_copy2d *copies, int n);

/* ---- timing on the library stream (hipEvents) -------------------------- */
void *plh_event_create(void);
int plh_event_record(void *ev);
float plh_event_elapsed_ms(void *start, void *stop); /* waits for stop */
void plh_event_destroy(void *ev);

/* ---- HIP graphs of the library stream ------------------------------------ */
/* Everything queued between begin and end (attention launches, event
 * records) is captured instead of run; plh_graph_launch replays it.  Decode
 * and prefill launches need no memset and allocate nothing once the library
 * workspace has been sized by one eager call of the same shape (decode split
 * partials; prefill chunk partials of split one-layer launches), so they can
 * be captured.  A later, larger call moves to a bigger workspace; the old one
 * stays allocated until plh_shutdown, so graphs captured earlier keep
 * replaying correctly. */
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
 * 0..pos.  Supported: every even head_dim up to 256 (model.c:408, 856; 64 and
 * 128 run tuned kernels, the others generic ones), n_heads % n_kv_heads == 0.  Any
 * finite q is handled: a q head with some |element| >= 2^15 is scaled by a
 * power of two before its fp16 split and the factor moves into its score
 * scale (exact). */
int plh_attn_decode(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                    int max_seq_len, int rope_type, int layer0,
                    int n_launch_layers, int pos, const float *q,
                    const float *k, const float *v, uint16_t *key_cache,
                    uint16_t *val_cache, const float *rope_cos,
                    const float *rope_sin, float *out);

/* ---- decode attention that also hands back the appended rows ------------- */
/* plh_attn_decode (q_norm = k_norm = NULL) or plh_attn_decode_qknorm with the
 * same arguments and results, whose kernel also writes the fp16 bits of the
 * appended row `pos` of every launched layer to k_rows and v_rows
 * ([n_launch_layers][n_kv_heads*head_dim] uint16_t each, layer li at
 * + li*kv_dim).  Every pointer may be any memory the device can access, such
 * as pinned host memory from plh_host_alloc: the gpu.h decode hook keeps q,
 * k, v, out and the rows in pinned staging and so needs no copy launches to
 * return model.c:822-826's cache rows to the host cache (gpu.c:691-699's
 * synchronous copy-back, for the attention block).  k_rows and v_rows must
 * not be null. */
int plh_attn_decode_rows(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                         int max_seq_len, int rope_type, int layer0,
                         int n_launch_layers, int pos, const float *q,
                         const float *k, const float *v, uint16_t *key_cache,
                         uint16_t *val_cache, const float *rope_cos,
                         const float *rope_sin, float *out, const float *q_norm,
                         const float *k_norm, float norm_eps, uint16_t *k_rows,
                         uint16_t *v_rows);

/* ---- decode attention without allocation -------------------------------- */
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): plh_attn_decode with the same arguments and results,
 * whose split partials live in a static device array of 16 MiB (each GPU the
 * library runs on holds it until the process ends) instead of the library
 * workspace.  It calls no hipMalloc / hipFree.  Returns -1 with a message
 * when a launch's partials would exceed the 16 MiB (very wide models: the
 * partials take n_units * min(G,16) * (head_dim+2) * 4 bytes, a few MiB at
 * the usual shapes).  Every call on a GPU shares that one array: calls that
 * overlap on one GPU race (the library's own stream serialises its calls). */
int plh_attn_decode_noalloc(int n_layers, int n_heads, int n_kv_heads, int head_dim,
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
 * (gpu.c:595-602): out[i] = vec_dot(row i of W, x).  Two summation orders
 * (plh_set_tuning key 10): the exact one is bit-identical to the reference's
 * fused dequantize + dot products in its x86-64 (AVX2 + FMA) build
 * (quant.c:390-452, 517-582, 627-659); the default fast one stages x as
 * fixed-point int8 digits (30 bits per 32-element block) and uses exact
 * integer dot products, within ~1e-7 of sum |w x| per output for ordinary
 * activations.  W is a d x n matrix, n a multiple of the block (256, 256,
 * 32).
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
/* plh_gemv with the forward pass's prologue and epilogues, in the
 * reference's order (rmsnorm tensor.c:425-492, matmul_bias tensor.c:256-264,
 * silu + elemwise_mul tensor.c:605-633, vec_add tensor.c:635-657):
 *     xn = rmsnorm(x, norm_w, norm_eps)  if norm_w (n <= 7680), else x
 *     v = vec_dot(row i, xn)
 *     v = v + bias[i]        if bias            (matmul_bias)
 *     v = v + 0.0f           if bias_zero       (matmul_bias with a zeroed bias)
 *     v = silu(gate[i]) * v  if gate            (hb = silu(hb) * hb2)
 *     out[i] = resid[i] + v  if resid, else v   (x += ...)
 * gate and resid may alias out (read before the row is written).  In the
 * exact order all but silu's expf are bit-identical to the reference; the
 * fast order also sums the rmsnorm squares as a tree. */
int plh_gemv_ex(int qtype, int n, int d, const void *dev, const float *x, float *out,
                const float *norm_w, float norm_eps, const float *bias, int bias_zero,
                const float *gate, const float *resid);

/* tensor.c:322-366 matmul_batch on the device: out[b*d + i] = vec_dot(row i
 * of W, x + b*n) for b < n_batch, each bit-identical to plh_gemv's exact
 * order (n_batch 1 runs plh_gemv itself, in the selected order). */
int plh_matmul_batch(int qtype, int n, int d, const void *dev, const float *x, int n_batch,
                     float *out);

/* The SwiGLU input of the FFN in one launch (model.c:906-916 -- gate and up
 * projections, silu, elemwise_mul): out[i] = silu(vec_dot(gate row i, xn)) *
 * vec_dot(up row i, xn), xn = rmsnorm(x, norm_w, norm_eps) when norm_w is
 * set (else x).  gate_dev / up_dev: packed copies of two d x n matrices of
 * the same type.  In the exact order the dot products and the norm are
 * bit-identical to the reference; silu uses the device expf. */
int plh_gemv_swiglu(int qtype, int n, int d, const void *gate_dev, const void *up_dev,
                    const float *x, float *out, const float *norm_w, float norm_eps);

/* ---- forward pass (model_forward_ex, model.c:746-925) --------------------- */
/* tensor.c:425-492 rmsnorm, bit-identical to the reference's x86-64 AVX2
 * build: out[i] = (x[i] * (1/sqrtf(sum(x^2)/n + eps))) * w[i], the sum in the
 * reference's eight-lane order.  Device pointers; out may alias x;
 * n <= 12288. */
int plh_rmsnorm(const float *x, const float *w, float *out, int n, float eps);
/* quant.c:265-276 dequantize_row on the device for F32, F16, Q4_0, Q8_0,
 * Q4_K and Q6_K rows (row: device pointer to the GGUF bytes), bit-identical. */
int plh_dequantize_row(int qtype, const void *row, float *out, int n);

/* One weight matrix of the forward pass: GGUF type id (Q4_K, Q6_K, Q8_0) and
 * its packed device copy (plh_gemv_upload). */
typedef struct {
    int qtype;
    const void *w;
} plh_matrix;

/* One layer (model.h:40-74 and the run state's dequantized copies,
 * model.c:644-707); fp32 device arrays. */
typedef struct {
    const float *attn_norm; /* [n_embd] */
    const float *ffn_norm;  /* [n_embd] */
    plh_matrix q, k, v, o, gate, up, down;
    const float *q_bias;    /* [n_heads*head_dim]; NULL adds zeros (model.c:781-782) */
    const float *k_bias;    /* [kv_dim] or NULL (model.c:792-795) */
    const float *v_bias;    /* [kv_dim] or NULL (model.c:797-800) */
    const float *o_bias;    /* [n_embd]; NULL adds zeros (model.c:895-896) */
    const float *q_norm;    /* [head_dim] Qwen3 QK-norm weights, or NULL */
    const float *k_norm;    /* [head_dim]; NULL exactly when q_norm is */
} plh_layer;

/* The model as plh_forward reads it (model.h:22-120 and model.c:545-556);
 * all pointers but `layers` are device memory. */
typedef struct {
    int n_layers, n_embd, n_ffn, n_heads, n_kv_heads, head_dim, vocab_size,
        max_seq_len, rope_type;
    float rms_norm_eps;
    int embd_type;            /* GGUF type of token_embd */
    const void *token_embd;   /* [vocab_size] GGUF rows of n_embd, as in the file */
    const float *output_norm; /* [n_embd] */
    plh_matrix output;        /* [vocab_size] x n_embd */
    uint16_t *key_cache;      /* the KV-cache layout above */
    uint16_t *val_cache;
    const float *rope_cos;    /* [max_seq_len][head_dim/2] */
    const float *rope_sin;
    const plh_layer *layers;  /* HOST array [n_layers] */
} plh_model;

/* Bytes of the activation workspace plh_forward needs for this model. */
size_t plh_forward_workspace_bytes(const plh_model *m);
/* Replaces model_forward_ex(m, token, pos, n_layers) (model.c:746-925): the
 * embedding row of `token`, every layer (rmsnorm, q/k/v projections and
 * biases, QK-norm if present, RoPE, FP16 append of row pos, attention over
 * rows 0..pos, output projection + bias + residual, rmsnorm, gate/up, silu,
 * down + residual), the final rmsnorm and the output projection into
 * logits [vocab_size] (device).  x_out (device, may be NULL) receives the
 * final normalised residual (the reference's s->x).  workspace: device,
 * plh_forward_workspace_bytes(m).  Even head dims up to 256; matrices Q4_K, Q6_K
 * or Q8_0.  Queued on the library stream. */
int plh_forward(const plh_model *m, int token, int pos, void *workspace, float *logits,
                float *x_out);
/* Replaces model_forward_prefill(m, tokens, n_tokens, start_pos)
 * (model.c:939-1144): the prompt tokens (HOST array) at positions
 * start_pos.., rows start_pos..start_pos+n_tokens-1 of every layer's caches
 * appended, logits and x_out of the last token only.  Chunks of up to 128
 * tokens go through each layer together (batched GEMVs reading each weight
 * about once per chunk, the prefill attention kernel); every (row, token)
 * product keeps the reference's arithmetic, q and output biases only when
 * present (model.c:1002-1017, 1095-1099).  Its activations live in a
 * library-owned buffer (grown on first use); `workspace` is not used. */
int plh_forward_prefill(const plh_model *m, const int *tokens, int n_tokens, int start_pos,
                        void *workspace, float *logits, float *x_out);

/* Tuning knobs (bench sweeps).  key 1: decode target workgroups per launch
 * (0 = default); key 2: decode contexts of at most this many positions are
 * not split (multiple of 128, 0 = default); key 3: GEMV rows per thread
 * (1, 2, 4, 8; 0 = default); key 4: plh_forward forms each rmsnorm in a
 * launch of its own (1) instead of inside the GEMVs that read it (0,
 * default); key 5: prefill launches with fewer q blocks than workgroup slots
 * split their heavy blocks into chunks of tiles merged afterwards (0
 * automatic, -1 never, 2, 4, 8 or 16 tiles per chunk); key 6: prefill
 * launches of at most one q block per CU run each block in a workgroup of 2
 * or 3 groups of 4 waves that share its tiles and merge in LDS (0
 * automatic, -1 never, 2 or 3 groups; head_dim 128 takes at most 2); key
 * 7: decode kernel (0 by shape, 1 split + combine, 2 stream-K with the merge
 * in the launch); key 8: stream-K workgroups (0 = by shape); key 9:
 * stream-K tiles in flight per wave (0 = default, 2, 3, 4); key 10: the
 * single-vector weight GEMVs (plh_gemv*, gpu_try_matmul, plh_forward) keep
 * the reference's x86 AVX2 summation order bit for bit (1) or use the
 * faster fixed-point-digit order (0, default: within ~1e-7 of sum |w x| per
 * output; the batched prompt GEMVs always keep the exact order); key 11:
 * stream-K groups whose producers share an XCD merge through its L2 (0 by
 * shape, 1 wherever the plan allows, -1 never: every merge device-wide);
 * key 14: the split decode kernel's partials are merged by each group's last
 * split inside the launch (0, default, where its splits share an XCD) or by
 * a combine launch (-1); key 15: plh_forward's attention launches add
 * workgroups, one per CU they leave idle, that load the weights of the
 * layer's o-projection, gate/up pair and down projection into the L2 of the
 * XCDs whose GEMV workgroups read them (0, default), of the first two only
 * (1), or none (-1); results are the same bits in every setting; key 17:
 * plh_forward runs a layer's q/k/v projections and its unsplit (short
 * context, no QK-norm, head_dim 64 or 128) attention in one launch, with 8
 * prefetch workgroups per XCD (0, default) or 8..31 of them, or in two
 * launches (-1); the same bits either way. */
int plh_set_tuning(int key, int value);

#ifdef __cplusplus
}
#endif

#endif /* PICOLM_HIP_H */
