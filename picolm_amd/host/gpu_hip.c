/*
 * gpu_hip.c -- picolm's gpu.h backend surface over libpicolm_hip (C11).
 *
 * The reference's Vulkan backend (gpu.c) keeps one global state, uploads
 * weights once and answers gpu_try_matmul synchronously with a staging copy,
 * a dispatch and a fence wait (gpu.c:579-702).  This backend does the same
 * for the attention block: one global state, the FP16 KV cache and RoPE
 * tables resident in HBM, and synchronous gpu_try_attention /
 * gpu_try_attention_prefill calls (copy in, one or two kernel launches, copy
 * out).  After every call the rows it appended are copied back into the
 * model's host cache, so the host cache stays authoritative and bit-equal to
 * the device one; a HIP failure after device state may have changed marks the
 * backend unavailable so that every later call falls back to the CPU.
 *
 * The weight GEMV (gpu_try_matmul, gpu.c:579-702) follows the Vulkan
 * backend's model too: gpu_upload_model uploads the projection matrices of
 * layers < PICOLM_GPU_LAYERS and the output matrix once (gpu.c:427-464),
 * packed for the kernels, and gpu_try_matmul finds a matrix by its host
 * pointer, copies x in, runs plh_gemv and copies out back.  Q4_K, Q6_K and
 * Q8_0 (the reference's three pipelines); other types return -1.
 *
 * Qwen3 layers (a non-null weights.layers[l].attn_q_norm, model.c:807-817
 * and 1029-1037) run on the device too: their dequantized QK-norm weights
 * (state.attn_q_norm_w[l] / attn_k_norm_w[l], model.c:657-670) are uploaded
 * with the tables and the *_qknorm entry points normalise q and k before
 * RoPE, with config.rms_norm_eps.
 *
 * When every matrix of the model is on the device, gpu_try_forward and
 * gpu_try_forward_prefill run the whole forward pass there (plh_forward):
 * the run state's dequantized norms and biases (model.c:644-707) and the raw
 * embedding rows are uploaded too; a call copies back the logits, the final
 * normalised residual (state.x) and the KV rows it appended.
 *
 * Built with USE_HIP; compiles against either this package's model.h or the
 * reference's (it reads only config.{n_embd, n_ffn, n_heads, n_kv_heads,
 * n_layers, vocab_size, max_seq_len, head_dim, rope_type, rms_norm_eps},
 * weights.{token_embd, type_token_embd, output, type_output} and
 * weights.layers[].{attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up,
 * ffn_down, their type_* fields, attn_q_norm, attn_q_b, attn_k_b, attn_v_b,
 * attn_output_b, type_attn_q_b, type_attn_output_b}, and state.{x, logits,
 * key_cache, val_cache, rope_cos, rope_sin, attn_norm_w, ffn_norm_w,
 * attn_q_norm_w, attn_k_norm_w, output_norm_w, attn_q_bias, attn_k_bias,
 * attn_v_bias, attn_output_bias}).
 */
#include "gpu_hip.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "picolm_hip.h"

/* One uploaded weight matrix: found by the caller's host pointer. */
typedef struct {
    const void *host;
    void *dev;
    int qtype, n, d;
} gpu_weight_t;

static struct {
    int inited;     /* plh_init succeeded */
    int uploaded;   /* caches and tables resident */
    int n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, n_embd;
    float norm_eps;
    int gpu_layers; /* layers < gpu_layers use the device */
    int fail_after; /* PICOLM_HIP_FAIL_AFTER: attention hook calls that succeed before an
                     * injected failure (-1: none) */
    uint16_t *d_key, *d_val;
    float *d_cos, *d_sin;
    unsigned char qkn[MAX_LAYERS]; /* layer has QK-norm */
    float *d_qn, *d_kn;            /* [n_layers][head_dim] QK-norm weights, or NULL */
    /* staging, sized for stage_tokens rows: device q|k|v (one block) and out;
     * pinned host h_in = q|k|v and h_out = out|key rows|val rows, so that a
     * call is one packed upload, the kernels and queued downloads with a
     * single synchronisation */
    float *d_q, *d_k, *d_v, *d_out;
    unsigned char *h_in, *h_out;
    int stage_tokens;
    gpu_weight_t *weights;          /* GEMV matrices */
    int n_weights, cap_weights;
    float *h_mx, *h_mout;           /* GEMV staging (pinned host memory, which the kernel
                                     * reads and writes directly): x [mx_cap], out [mout_cap] */
    int mx_cap, mout_cap;
    /* whole forward pass (gpu_try_forward): NULL model when unavailable */
    plh_model fwd;
    plh_layer fwd_layers[MAX_LAYERS];
    float *d_fwd_vecs;              /* norms and biases, one block */
    void *d_embd;                   /* raw token_embd rows */
    void *d_fwd_ws;                 /* plh_forward workspace */
    float *d_x;
    /* copy-back staging (pinned host memory): logits [vocab] (the output
     * GEMV writes them there itself), x [n_embd], then the key rows and the
     * val rows a call appended, [n_layers][n][kv_dim] each */
    unsigned char *h_fwd;
    size_t fwd_cap;
    int fwd_ready;
} gs;

static int env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    return atoi(s);
}

static void backend_lost(const char *what) {
    fprintf(stderr, "gpu_hip: %s failed (%s); attention stays on the CPU from now on\n", what,
            plh_last_error());
    gs.uploaded = 0;
}

/* Fault injection for the fallback tests (PICOLM_HIP_FAIL_AFTER=N): the
 * attention hook call after N successful ones fails as a HIP error after its
 * kernels would: the device cache already holds the new rows, the host cache
 * does not, and the backend is lost, so the caller's CPU block runs that layer
 * and every later one.  Returns 1 for the failing call. */
static int injected_failure(void) {
    if (gs.fail_after < 0) return 0;
    if (gs.fail_after-- > 0) return 0;
    fprintf(stderr, "gpu_hip: injected failure (PICOLM_HIP_FAIL_AFTER)\n");
    return 1;
}

int gpu_init(const model_t *m) {
    if (gs.inited) return 0;
    if (env_int("PICOLM_HIP_DISABLE", 0)) return -1;
    const model_config_t *c = &m->config;
    /* every head_dim the reference runs (even, at most 256: its acc[256],
     * model.c:856); 64 and 128 have tuned kernels, the others a generic one */
    if (c->head_dim < 2 || c->head_dim > 256 || c->head_dim % 2) {
        fprintf(stderr, "gpu_hip: head_dim %d has no kernel, attention stays on the CPU\n",
                c->head_dim);
        return -1;
    }
    if (c->n_layers < 1 || c->n_layers > MAX_LAYERS) return -1;
    if (plh_init(env_int("PICOLM_HIP_DEVICE", 0)) != 0) {
        fprintf(stderr, "gpu_hip: %s\n", plh_last_error());
        return -1;
    }
    /* PICOLM_HIP_GEMV_EXACT=1: the weight GEMVs keep the reference's x86 AVX2
     * summation order bit for bit (gpu_try_matmul then equals the CPU matmul
     * exactly); by default they use the faster order, within the forward
     * pass's tolerance. */
    if (plh_set_tuning(10, env_int("PICOLM_HIP_GEMV_EXACT", 0) ? 1 : 0) != 0) {
        fprintf(stderr, "gpu_hip: %s\n", plh_last_error());
        return -1;
    }
    gs.inited = 1;
    gs.n_layers = c->n_layers;
    gs.n_heads = c->n_heads;
    gs.n_kv_heads = c->n_kv_heads;
    gs.head_dim = c->head_dim;
    gs.max_seq_len = c->max_seq_len;
    gs.rope_type = (int)c->rope_type;
    gs.n_embd = c->n_embd;
    gs.norm_eps = c->rms_norm_eps;
    gs.gpu_layers = env_int("PICOLM_GPU_LAYERS", c->n_layers);
    gs.fail_after = env_int("PICOLM_HIP_FAIL_AFTER", -1);
    return 0;
}

static size_t cache_bytes(void) {
    return (size_t)gs.n_layers * (size_t)gs.max_seq_len * (size_t)gs.n_kv_heads *
           (size_t)gs.head_dim * sizeof(uint16_t);
}

static void free_stage(void) {
    plh_free(gs.d_q);
    plh_free(gs.d_out);
    plh_host_free(gs.h_in);
    plh_host_free(gs.h_out);
    gs.d_q = gs.d_k = gs.d_v = gs.d_out = NULL;
    gs.h_in = gs.h_out = NULL;
    gs.stage_tokens = 0;
}

static int ensure_stage(int n_tokens) {
    if (n_tokens <= gs.stage_tokens) return 0;
    free_stage();
    size_t q_dim = (size_t)gs.n_heads * gs.head_dim;
    size_t kv_dim = (size_t)gs.n_kv_heads * gs.head_dim;
    size_t q4 = (q_dim + 3) & ~(size_t)3; /* the device output stride */
    size_t stride = (size_t)gs.n_embd > q4 ? (size_t)gs.n_embd : q4;
    size_t in_bytes = (size_t)n_tokens * (q_dim + 2 * kv_dim) * sizeof(float);
    size_t out_bytes = (size_t)n_tokens * stride * sizeof(float);
    size_t rows_bytes = 2 * (size_t)n_tokens * kv_dim * sizeof(uint16_t);
    gs.d_q = (float *)plh_malloc(in_bytes);
    gs.d_out = (float *)plh_malloc(out_bytes);
    gs.h_in = (unsigned char *)plh_host_alloc(in_bytes);
    gs.h_out = (unsigned char *)plh_host_alloc(out_bytes + rows_bytes);
    if (!gs.d_q || !gs.d_out || !gs.h_in || !gs.h_out) {
        free_stage();
        return -1;
    }
    gs.d_k = gs.d_q + (size_t)n_tokens * q_dim;
    gs.d_v = gs.d_k + (size_t)n_tokens * kv_dim;
    gs.stage_tokens = n_tokens;
    return 0;
}

/* q, k, v of n rows into pinned staging, then one upload to d_q|d_k|d_v
 * (queued).  The device q block is n rows of q_dim, so k and v follow it. */
static int stage_in(int n, const float *q, const float *k, const float *v) {
    const size_t qb = (size_t)n * gs.n_heads * gs.head_dim * sizeof(float);
    const size_t kvb = (size_t)n * gs.n_kv_heads * gs.head_dim * sizeof(float);
    memcpy(gs.h_in, q, qb);
    memcpy(gs.h_in + qb, k, kvb);
    memcpy(gs.h_in + qb + kvb, v, kvb);
    gs.d_k = gs.d_q + (size_t)n * gs.n_heads * gs.head_dim;
    gs.d_v = gs.d_k + (size_t)n * gs.n_kv_heads * gs.head_dim;
    return plh_memcpy_htod_async(gs.d_q, gs.h_in, qb + 2 * kvb);
}

/* Copies out (out_bytes from d_out) and rows [r0, r0+n) of layer `layer` of
 * both device caches into h_out, then synchronises: up to 8 MB in all by one
 * copy kernel (531-546 against 559-593 us per call for a 512-token TinyLlama
 * prompt, 4.5 MB), larger ones as three DMA copies, which the kernel's PCIe
 * stores did not beat (4.5-4.7 ms per call either way for 32 MB). */
static int stage_out(size_t out_bytes, int layer, int r0, int n) {
    const size_t kv_dim = (size_t)gs.n_kv_heads * gs.head_dim;
    const size_t off = ((size_t)layer * gs.max_seq_len + (size_t)r0) * kv_dim;
    const size_t rb = (size_t)n * kv_dim * sizeof(uint16_t);
    if (out_bytes + 2 * rb <= ((size_t)8 << 20)) {
        const plh_copy2d back[3] = {
            {gs.h_out, out_bytes, gs.d_out, out_bytes, out_bytes, 1},
            {gs.h_out + out_bytes, rb, gs.d_key + off, rb, rb, 1},
            {gs.h_out + out_bytes + rb, rb, gs.d_val + off, rb, rb, 1},
        };
        if (plh_copy2d_batch_async(back, 3) != 0) return -1;
    } else if (plh_memcpy_dtoh_async(gs.h_out, gs.d_out, out_bytes) != 0 ||
               plh_memcpy_dtoh_async(gs.h_out + out_bytes, gs.d_key + off, rb) != 0 ||
               plh_memcpy_dtoh_async(gs.h_out + out_bytes + rb, gs.d_val + off, rb) != 0) {
        return -1;
    }
    return plh_synchronize();
}

/* The staged rows of stage_out into the host caches. */
static void rows_from_stage(const model_t *m, size_t out_bytes, int layer, int r0, int n) {
    const size_t kv_dim = (size_t)gs.n_kv_heads * gs.head_dim;
    const size_t off = ((size_t)layer * gs.max_seq_len + (size_t)r0) * kv_dim;
    const size_t rb = (size_t)n * kv_dim * sizeof(uint16_t);
    memcpy(m->state.key_cache + off, gs.h_out + out_bytes, rb);
    memcpy(m->state.val_cache + off, gs.h_out + out_bytes + rb, rb);
}

/* Per-layer QK-norm weights, as the host dequantized them at load
 * (model.c:657-670); layers without attn_q_norm keep the plain entry points. */
static int upload_qk_norm(const model_t *m) {
    int any = 0;
    for (int l = 0; l < gs.n_layers; l++) {
        gs.qkn[l] = m->weights.layers[l].attn_q_norm != NULL;
        any |= gs.qkn[l];
    }
    if (!any) return 0;
    size_t row = (size_t)gs.head_dim * sizeof(float);
    gs.d_qn = (float *)plh_malloc((size_t)gs.n_layers * row);
    gs.d_kn = (float *)plh_malloc((size_t)gs.n_layers * row);
    if (!gs.d_qn || !gs.d_kn) return -1;
    for (int l = 0; l < gs.n_layers; l++) {
        if (!gs.qkn[l]) continue;
        if (!m->state.attn_q_norm_w[l] || !m->state.attn_k_norm_w[l]) return -1;
        size_t off = (size_t)l * gs.head_dim;
        if (plh_memcpy_htod(gs.d_qn + off, m->state.attn_q_norm_w[l], row) != 0 ||
            plh_memcpy_htod(gs.d_kn + off, m->state.attn_k_norm_w[l], row) != 0)
            return -1;
    }
    return 0;
}

/* Uploads one projection matrix (d rows of n) if the GEMV has a kernel for
 * its type; matrices it cannot run stay on the CPU path. */
static int upload_weight(const void *host, int qtype, int d, int n) {
    if (!host) return 0;
    size_t bytes = plh_gemv_packed_bytes(qtype, n, d);
    if (bytes == 0) return 0;
    if (gs.n_weights == gs.cap_weights) {
        int cap = gs.cap_weights ? 2 * gs.cap_weights : 64;
        gpu_weight_t *w = (gpu_weight_t *)realloc(gs.weights, (size_t)cap * sizeof *w);
        if (!w) return -1;
        gs.weights = w;
        gs.cap_weights = cap;
    }
    void *dev = plh_malloc(bytes);
    if (!dev) return -1;
    if (plh_gemv_upload(qtype, n, d, host, dev) != 0) {
        plh_free(dev);
        return -1;
    }
    gpu_weight_t *w = &gs.weights[gs.n_weights++];
    w->host = host;
    w->dev = dev;
    w->qtype = qtype;
    w->n = n;
    w->d = d;
    if (n > gs.mx_cap) gs.mx_cap = n;
    if (d > gs.mout_cap) gs.mout_cap = d;
    return 0;
}

/* gpu.c:447-458: the seven projections of layers < gpu_layers, then the
 * output matrix.  attn_q is uploaded with the q_dim = n_heads*head_dim rows
 * that model.c:779-781 multiplies with; gpu.c:451 passes n_embd, the same
 * number for every model the reference loads (head_dim = n_embd / n_heads,
 * model.c:408), but for a hand-built layout it would read past the host
 * tensor when q_dim < n_embd. */
static int upload_weights(const model_t *m) {
    const model_config_t *c = &m->config;
    int kv_dim = c->n_kv_heads * c->head_dim, q_dim = c->n_heads * c->head_dim;
    for (int l = 0; l < gs.gpu_layers && l < c->n_layers; l++) {
        const layer_weights_t *lw = &m->weights.layers[l];
        if (upload_weight(lw->attn_q, (int)lw->type_attn_q, q_dim, c->n_embd) ||
            upload_weight(lw->attn_k, (int)lw->type_attn_k, kv_dim, c->n_embd) ||
            upload_weight(lw->attn_v, (int)lw->type_attn_v, kv_dim, c->n_embd) ||
            upload_weight(lw->attn_output, (int)lw->type_attn_output, c->n_embd, q_dim) ||
            upload_weight(lw->ffn_gate, (int)lw->type_ffn_gate, c->n_ffn, c->n_embd) ||
            upload_weight(lw->ffn_up, (int)lw->type_ffn_up, c->n_ffn, c->n_embd) ||
            upload_weight(lw->ffn_down, (int)lw->type_ffn_down, c->n_embd, c->n_ffn))
            return -1;
    }
    if (gs.gpu_layers > 0 &&
        upload_weight(m->weights.output, (int)m->weights.type_output, c->vocab_size,
                      c->n_embd))
        return -1;
    if (gs.n_weights > 0) {
        gs.h_mx = (float *)plh_host_alloc((size_t)gs.mx_cap * sizeof(float));
        gs.h_mout = (float *)plh_host_alloc((size_t)gs.mout_cap * sizeof(float));
        if (!gs.h_mx || !gs.h_mout) return -1;
    }
    return 0;
}

static void free_weights(void) {
    for (int i = 0; i < gs.n_weights; i++) plh_free(gs.weights[i].dev);
    free(gs.weights);
    plh_host_free(gs.h_mx);
    plh_host_free(gs.h_mout);
    gs.weights = NULL;
    gs.n_weights = gs.cap_weights = 0;
    gs.h_mx = gs.h_mout = NULL;
    gs.mx_cap = gs.mout_cap = 0;
}

static const gpu_weight_t *find_weight(const void *host) {
    for (int i = 0; i < gs.n_weights; i++)
        if (gs.weights[i].host == host) return &gs.weights[i];
    return NULL;
}

static int fwd_matrix(plh_matrix *pm, const void *host, gguf_type_t qtype, int n, int d) {
    const gpu_weight_t *w = find_weight(host);
    if (!w || w->qtype != (int)qtype || w->n != n || w->d != d) return -1;
    pm->qtype = w->qtype;
    pm->w = w->dev;
    return 0;
}

/* Bytes of one embedding row for the types plh_forward dequantises on the
 * device (quant.c:283-325). */
static size_t embd_row_bytes(gguf_type_t t, int n) {
    switch ((int)t) {
        case GGUF_TYPE_F32: return (size_t)n * 4;
        case GGUF_TYPE_F16: return (size_t)n * 2;
        case GGUF_TYPE_Q4_0: return n % 32 ? 0 : (size_t)(n / 32) * 18;
        case GGUF_TYPE_Q8_0: return n % 32 ? 0 : (size_t)(n / 32) * 34;
        case GGUF_TYPE_Q4_K: return n % 256 ? 0 : (size_t)(n / 256) * 144;
        case GGUF_TYPE_Q6_K: return n % 256 ? 0 : (size_t)(n / 256) * 210;
        default: return 0;
    }
}

static void free_forward(void) {
    plh_free(gs.d_fwd_vecs);
    plh_free(gs.d_embd);
    plh_free(gs.d_fwd_ws);
    plh_free(gs.d_x);
    plh_host_free(gs.h_fwd);
    gs.d_fwd_vecs = NULL;
    gs.d_embd = gs.d_fwd_ws = NULL;
    gs.d_x = NULL;
    gs.h_fwd = NULL;
    gs.fwd_cap = 0;
    gs.fwd_ready = 0;
}

/* The device model of gpu_try_forward: every layer's seven projections and
 * the output matrix must already be uploaded (GEMV types), the embedding of
 * a type the device dequantises, the biases fp32 (the reference adds the
 * pre-dequantized q and output biases through dequantize_row of their file
 * type, model.c:781-782, which only an F32 file type leaves intact).  Returns
 * 0 with gs.fwd_ready set, 1 when the model does not qualify (the per-op
 * hooks still run), -1 on a device failure. */
static int upload_forward(const model_t *m) {
    const model_config_t *c = &m->config;
    const model_weights_t *w = &m->weights;
    const run_state_t *st = &m->state;
    const int E = c->n_embd, F = c->n_ffn, Q = c->n_heads * c->head_dim;
    const int KV = c->n_kv_heads * c->head_dim;
    if (gs.gpu_layers < c->n_layers || E > 12288 || !w->token_embd || !st->logits || !st->x)
        return 1;
    /* The reference's loader sets head_dim = n_embd / n_heads (model.c:408),
     * so its forward pass only ever runs q_dim == n_embd (its q and xb buffers
     * hold n_embd floats, model.c:568-571); other layouts keep the CPU path. */
    if (Q != E) return 1;
    const size_t rb = embd_row_bytes(w->type_token_embd, E);
    if (rb == 0) return 1;
    plh_model *pm = &gs.fwd;
    memset(pm, 0, sizeof *pm);
    if (fwd_matrix(&pm->output, w->output, w->type_output, E, c->vocab_size)) return 1;
    /* fp32 vectors: per layer attn_norm, ffn_norm [E], q_bias [Q], k_bias,
     * v_bias [KV], o_bias [E]; then output_norm [E] */
    const size_t per_layer = (size_t)3 * E + Q + 2 * (size_t)KV;
    for (int l = 0; l < c->n_layers; l++) {
        const layer_weights_t *lw = &w->layers[l];
        plh_layer *pl = &gs.fwd_layers[l];
        memset(pl, 0, sizeof *pl);
        if (fwd_matrix(&pl->q, lw->attn_q, lw->type_attn_q, E, Q) ||
            fwd_matrix(&pl->k, lw->attn_k, lw->type_attn_k, E, KV) ||
            fwd_matrix(&pl->v, lw->attn_v, lw->type_attn_v, E, KV) ||
            fwd_matrix(&pl->o, lw->attn_output, lw->type_attn_output, Q, E) ||
            fwd_matrix(&pl->gate, lw->ffn_gate, lw->type_ffn_gate, E, F) ||
            fwd_matrix(&pl->up, lw->ffn_up, lw->type_ffn_up, E, F) ||
            fwd_matrix(&pl->down, lw->ffn_down, lw->type_ffn_down, F, E))
            return 1;
        if ((lw->attn_q_b && lw->type_attn_q_b != GGUF_TYPE_F32) ||
            (lw->attn_output_b && lw->type_attn_output_b != GGUF_TYPE_F32))
            return 1;
        if (!st->attn_norm_w[l] || !st->ffn_norm_w[l] || !st->attn_q_bias[l] ||
            !st->attn_output_bias[l] || (lw->attn_k_b && !st->attn_k_bias[l]) ||
            (lw->attn_v_b && !st->attn_v_bias[l]))
            return 1;
    }
    if (!st->output_norm_w) return 1;
    size_t nvec = per_layer * (size_t)c->n_layers + (size_t)E;
    gs.d_fwd_vecs = (float *)plh_malloc(nvec * sizeof(float));
    gs.d_embd = plh_malloc(rb * (size_t)c->vocab_size);
    gs.d_x = (float *)plh_malloc((size_t)E * sizeof(float));
    if (!gs.d_fwd_vecs || !gs.d_embd || !gs.d_x) return -1;
    if (plh_memcpy_htod(gs.d_embd, w->token_embd, rb * (size_t)c->vocab_size)) return -1;
    float *dv = gs.d_fwd_vecs;
#define PUT(dst, src, count)                                                   \
    do {                                                                       \
        if (plh_memcpy_htod(dv, (src), (size_t)(count) * sizeof(float))) return -1; \
        (dst) = dv;                                                            \
        dv += (count);                                                         \
    } while (0)
    for (int l = 0; l < c->n_layers; l++) {
        const layer_weights_t *lw = &w->layers[l];
        plh_layer *pl = &gs.fwd_layers[l];
        PUT(pl->attn_norm, st->attn_norm_w[l], E);
        PUT(pl->ffn_norm, st->ffn_norm_w[l], E);
        /* q and output biases: the run state's buffers, zeros when the
         * layer has none -- added either way, as model_forward_ex does */
        PUT(pl->q_bias, st->attn_q_bias[l], Q);
        PUT(pl->o_bias, st->attn_output_bias[l], E);
        if (lw->attn_k_b) PUT(pl->k_bias, st->attn_k_bias[l], KV);
        else dv += KV;
        if (lw->attn_v_b) PUT(pl->v_bias, st->attn_v_bias[l], KV);
        else dv += KV;
        if (gs.qkn[l]) {
            pl->q_norm = gs.d_qn + (size_t)l * c->head_dim;
            pl->k_norm = gs.d_kn + (size_t)l * c->head_dim;
        }
    }
    PUT(pm->output_norm, st->output_norm_w, E);
#undef PUT
    pm->n_layers = c->n_layers;
    pm->n_embd = E;
    pm->n_ffn = F;
    pm->n_heads = c->n_heads;
    pm->n_kv_heads = c->n_kv_heads;
    pm->head_dim = c->head_dim;
    pm->vocab_size = c->vocab_size;
    pm->max_seq_len = c->max_seq_len;
    pm->rope_type = (int)c->rope_type;
    pm->rms_norm_eps = c->rms_norm_eps;
    pm->embd_type = (int)w->type_token_embd;
    pm->token_embd = gs.d_embd;
    pm->key_cache = gs.d_key;
    pm->val_cache = gs.d_val;
    pm->rope_cos = gs.d_cos;
    pm->rope_sin = gs.d_sin;
    pm->layers = gs.fwd_layers;
    gs.d_fwd_ws = plh_malloc(plh_forward_workspace_bytes(pm));
    if (!gs.d_fwd_ws) return -1;
    gs.fwd_ready = 1;
    return 0;
}

int gpu_upload_model(const model_t *m) {
    if (!gs.inited) return -1;
    if (gs.uploaded) return 0;
    size_t tab = (size_t)gs.max_seq_len * (size_t)(gs.head_dim / 2) * sizeof(float);
    gs.d_key = (uint16_t *)plh_malloc(cache_bytes());
    gs.d_val = (uint16_t *)plh_malloc(cache_bytes());
    gs.d_cos = (float *)plh_malloc(tab);
    gs.d_sin = (float *)plh_malloc(tab);
    if (!gs.d_key || !gs.d_val || !gs.d_cos || !gs.d_sin || ensure_stage(1) != 0) {
        fprintf(stderr, "gpu_hip: out of device memory: %s\n", plh_last_error());
        return -1;
    }
    /* The tables are the host's own (model.c:545-556), so device RoPE is
     * bit-identical; the cache mirrors whatever the host holds. */
    if (plh_memcpy_htod(gs.d_cos, m->state.rope_cos, tab) != 0 ||
        plh_memcpy_htod(gs.d_sin, m->state.rope_sin, tab) != 0 ||
        plh_memcpy_htod(gs.d_key, m->state.key_cache, cache_bytes()) != 0 ||
        plh_memcpy_htod(gs.d_val, m->state.val_cache, cache_bytes()) != 0) {
        fprintf(stderr, "gpu_hip: upload failed: %s\n", plh_last_error());
        return -1;
    }
    if (upload_qk_norm(m) != 0) {
        fprintf(stderr, "gpu_hip: QK-norm weight upload failed: %s\n", plh_last_error());
        return -1;
    }
    if (env_int("PICOLM_HIP_MATMUL", 1) && upload_weights(m) != 0) {
        /* like a failed tensor upload in gpu.c:441-443: the matmuls stay on
         * the CPU, attention still runs on the device */
        fprintf(stderr, "gpu_hip: weight upload failed (%s); matmuls stay on the CPU\n",
                plh_last_error());
        free_weights();
    }
    if (gs.n_weights > 0 && env_int("PICOLM_HIP_FORWARD", 1)) {
        const int rc = upload_forward(m);
        if (rc != 0) free_forward();
        if (rc < 0)
            fprintf(stderr, "gpu_hip: forward-pass upload failed (%s); per-op offload only\n",
                    plh_last_error());
    }
    gs.uploaded = 1;
    return 0;
}

int gpu_available(void) { return gs.inited && gs.uploaded; }

int gpu_try_matmul(float *out, const float *x, const void *W, int n, int d,
                   gguf_type_t qtype) {
    if (!gpu_available() || !W || !x || !out) return -1;
    const gpu_weight_t *w = NULL;
    for (int i = 0; i < gs.n_weights; i++)   /* gpu.c:583-591: lookup by host pointer */
        if (gs.weights[i].host == W) {
            w = &gs.weights[i];
            break;
        }
    if (!w || w->qtype != (int)qtype || w->n != n || w->d != d) return -1;
    /* x in and out back through pinned staging that the kernel reads and
     * writes itself: one launch and one synchronisation, no copy commands
     * (the Vulkan backend copies through its own staging, gpu.c:606-699) */
    memcpy(gs.h_mx, x, (size_t)n * sizeof(float));
    if (plh_gemv(w->qtype, n, d, w->dev, gs.h_mx, gs.h_mout) != 0 || plh_synchronize() != 0)
        return -1; /* nothing but staging changed: the CPU path stays intact */
    memcpy(out, gs.h_mout, (size_t)d * sizeof(float));
    return 0;
}

void gpu_shutdown(void) {
    if (gs.inited) {
        plh_synchronize();
        plh_free(gs.d_key);
        plh_free(gs.d_val);
        plh_free(gs.d_cos);
        plh_free(gs.d_sin);
        plh_free(gs.d_qn);
        plh_free(gs.d_kn);
        free_stage();
        free_forward();
        free_weights();
        plh_shutdown();
    }
    memset(&gs, 0, sizeof gs);
}

static int same_shape(const model_t *m) {
    const model_config_t *c = &m->config;
    return c->n_layers == gs.n_layers && c->n_heads == gs.n_heads &&
           c->n_kv_heads == gs.n_kv_heads && c->head_dim == gs.head_dim &&
           c->max_seq_len == gs.max_seq_len && (int)c->rope_type == gs.rope_type &&
           c->n_embd == gs.n_embd && c->rms_norm_eps == gs.norm_eps;
}

int gpu_try_attention(model_t *m, int layer, int pos, float *q, float *k, const float *v,
                      float *out) {
    if (!gpu_available() || !same_shape(m)) return -1;
    if (layer < 0 || layer >= gs.n_layers || layer >= gs.gpu_layers) return -1;
    if (pos < 0 || pos >= gs.max_seq_len) return -1;
    /* One token's q, k, v, out and cache rows are a few KiB: the kernels read
     * and write them in the pinned staging itself (pinned host memory is
     * device-accessible at the same address), so a call is one launch (two
     * with a split combine) and one synchronisation, no copy commands. */
    const size_t q_bytes = (size_t)gs.n_heads * gs.head_dim * sizeof(float);
    const size_t kv_bytes = (size_t)gs.n_kv_heads * gs.head_dim * sizeof(float);
    const size_t row_bytes = (size_t)gs.n_kv_heads * gs.head_dim * sizeof(uint16_t);
    memcpy(gs.h_in, q, q_bytes);
    memcpy(gs.h_in + q_bytes, k, kv_bytes);
    memcpy(gs.h_in + q_bytes + kv_bytes, v, kv_bytes);
    const float *hq = (const float *)gs.h_in;
    const float *hk = (const float *)(gs.h_in + q_bytes);
    const float *hv = (const float *)(gs.h_in + q_bytes + kv_bytes);
    const size_t off = (size_t)layer * gs.head_dim;
    const int qkn = gs.qkn[layer];
    int rc = plh_attn_decode_rows(gs.n_layers, gs.n_heads, gs.n_kv_heads, gs.head_dim,
                                  gs.max_seq_len, gs.rope_type, layer, 1, pos, hq, hk, hv,
                                  gs.d_key, gs.d_val, gs.d_cos, gs.d_sin, (float *)gs.h_out,
                                  qkn ? gs.d_qn + off : NULL, qkn ? gs.d_kn + off : NULL,
                                  gs.norm_eps, (uint16_t *)(gs.h_out + q_bytes),
                                  (uint16_t *)(gs.h_out + q_bytes + row_bytes));
    if (rc == 0) rc = plh_synchronize();
    if (rc != 0 || injected_failure()) {
        backend_lost("plh_attn_decode_rows");
        return -1;
    }
    memcpy(out, gs.h_out, q_bytes);
    rows_from_stage(m, q_bytes, layer, pos, 1);
    return 0;
}

int gpu_try_attention_prefill(model_t *m, int layer, int start_pos, int n_tokens, float *q,
                              float *k, const float *v, float *out) {
    if (!gpu_available() || !same_shape(m)) return -1;
    if (layer < 0 || layer >= gs.n_layers || layer >= gs.gpu_layers) return -1;
    if (start_pos < 0 || n_tokens < 0 || (long)start_pos + n_tokens > (long)gs.max_seq_len)
        return -1;
    if (n_tokens == 0) return 0;
    if (ensure_stage(n_tokens) != 0) {
        backend_lost("staging allocation");
        return -1;
    }
    size_t q_dim = (size_t)gs.n_heads * gs.head_dim;
    size_t stride = (size_t)gs.n_embd; /* out row bi at out + bi*n_embd (model.c:1057) */
    if (stride < q_dim) return -1;
    if (stage_in(n_tokens, q, k, v) != 0) {
        backend_lost("staging copy"); /* as in gpu_try_attention */
        return -1;
    }
    int dev_stride = (int)((q_dim + 3) & ~(size_t)3);
    int rc;
    if (gs.qkn[layer]) {
        size_t off = (size_t)layer * gs.head_dim;
        rc = plh_attn_prefill_qknorm(gs.n_layers, gs.n_heads, gs.n_kv_heads, gs.head_dim,
                                     gs.max_seq_len, gs.rope_type, layer, 1, start_pos,
                                     n_tokens, gs.d_q, gs.d_k, gs.d_v, gs.d_key, gs.d_val,
                                     gs.d_cos, gs.d_sin, gs.d_out, dev_stride, gs.d_qn + off,
                                     gs.d_kn + off, gs.norm_eps);
    } else {
        rc = plh_attn_prefill(gs.n_layers, gs.n_heads, gs.n_kv_heads, gs.head_dim,
                              gs.max_seq_len, gs.rope_type, layer, 1, start_pos, n_tokens,
                              gs.d_q, gs.d_k, gs.d_v, gs.d_key, gs.d_val, gs.d_cos, gs.d_sin,
                              gs.d_out, dev_stride);
    }
    if (rc != 0 || injected_failure()) {
        backend_lost("plh_attn_prefill");
        return -1;
    }
    const size_t out_bytes = (size_t)n_tokens * dev_stride * sizeof(float);
    if (stage_out(out_bytes, layer, start_pos, n_tokens) != 0) {
        backend_lost("copy back");
        return -1;
    }
    const float *staged = (const float *)gs.h_out;
    if ((size_t)dev_stride == stride) {
        memcpy(out, staged, out_bytes);
    } else {
        for (int bi = 0; bi < n_tokens; bi++)
            memcpy(out + (size_t)bi * stride, staged + (size_t)bi * dev_stride,
                   q_dim * sizeof(float));
    }
    rows_from_stage(m, out_bytes, layer, start_pos, n_tokens);
    return 0;
}

/* Rows 0..n_pos-1 of the layers the device handles (l < gpu_layers), one
 * strided copy per cache (host and device caches share the layout
 * [layer][max_seq_len][kv_dim]).  The other layers' rows exist only in the
 * host cache (their CPU block appends them there), so they are neither
 * overwritten by a download nor needed on the device. */
static int kv_copy(const model_t *m, int n_pos, int to_host) {
    if (!gpu_available() || !same_shape(m) || n_pos < 0 || n_pos > gs.max_seq_len) return -1;
    const size_t kv_dim = (size_t)gs.n_kv_heads * gs.head_dim;
    const size_t width = (size_t)n_pos * kv_dim * sizeof(uint16_t);
    const size_t pitch = (size_t)gs.max_seq_len * kv_dim * sizeof(uint16_t);
    const size_t layers = (size_t)(gs.gpu_layers < gs.n_layers ? gs.gpu_layers : gs.n_layers);
    int rc;
    if (to_host)
        rc = plh_memcpy2d_dtoh(m->state.key_cache, pitch, gs.d_key, pitch, width, layers) ||
             plh_memcpy2d_dtoh(m->state.val_cache, pitch, gs.d_val, pitch, width, layers);
    else
        rc = plh_memcpy2d_htod(gs.d_key, pitch, m->state.key_cache, pitch, width, layers) ||
             plh_memcpy2d_htod(gs.d_val, pitch, m->state.val_cache, pitch, width, layers);
    if (rc) {
        backend_lost(to_host ? "kv download" : "kv upload");
        return -1;
    }
    return 0;
}

int gpu_kv_download(const model_t *m, int n_pos) { return kv_copy(m, n_pos, 1); }

int gpu_kv_upload(const model_t *m, int n_pos) { return kv_copy(m, n_pos, 0); }

/* h_fwd sized for the logits, x and n positions' rows: grown on demand,
 * NULL (the CPU path runs) when the pinned allocation fails. */
static float *forward_stage(int n) {
    const size_t kv_dim = (size_t)gs.n_kv_heads * gs.head_dim;
    const size_t need = ((size_t)gs.fwd.vocab_size + (size_t)gs.n_embd) * sizeof(float) +
                        (size_t)2 * gs.n_layers * n * kv_dim * sizeof(uint16_t);
    if (need > gs.fwd_cap) {
        plh_host_free(gs.h_fwd);
        gs.h_fwd = (unsigned char *)plh_host_alloc(need);
        gs.fwd_cap = gs.h_fwd ? need : 0;
    }
    return (float *)gs.h_fwd;
}

/* After plh_forward(_prefill) has written the logits into h_fwd: x and the
 * rows of positions pos0..pos0+n-1 of every layer into h_fwd by one copy
 * kernel (x, then one strided copy per cache), one synchronisation, then the
 * host state and caches filled from the staging. */
static int forward_done(model_t *m, int pos0, int n) {
    const model_config_t *c = &m->config;
    const size_t kv_dim = (size_t)gs.n_kv_heads * gs.head_dim;
    const size_t off = (size_t)pos0 * kv_dim;
    const size_t pitch = (size_t)gs.max_seq_len * kv_dim * sizeof(uint16_t);
    const size_t width = (size_t)n * kv_dim * sizeof(uint16_t);
    const size_t lb = (size_t)c->vocab_size * sizeof(float), xb = (size_t)c->n_embd * sizeof(float);
    const size_t rb = width * (size_t)gs.n_layers;
    unsigned char *hx = gs.h_fwd + lb, *hk = hx + xb, *hv = hk + rb;
    const plh_copy2d back[3] = {
        {hx, xb, gs.d_x, xb, xb, 1},
        {hk, width, gs.d_key + off, pitch, width, (size_t)gs.n_layers},
        {hv, width, gs.d_val + off, pitch, width, (size_t)gs.n_layers},
    };
    if (plh_copy2d_batch_async(back, 3) || plh_synchronize()) {
        backend_lost("copy back");
        return -1;
    }
    memcpy(m->state.logits, gs.h_fwd, lb);
    memcpy(m->state.x, hx, xb);
    const size_t lstride = (size_t)gs.max_seq_len * kv_dim;
    for (int l = 0; l < gs.n_layers; l++) {
        memcpy(m->state.key_cache + l * lstride + off, hk + l * width, width);
        memcpy(m->state.val_cache + l * lstride + off, hv + l * width, width);
    }
    return 0;
}

int gpu_try_forward(model_t *m, int token, int pos) {
    if (!gpu_available() || !gs.fwd_ready || !same_shape(m)) return -1;
    if (token < 0 || token >= m->config.vocab_size || pos < 0 || pos >= gs.max_seq_len) return -1;
    float *logits = forward_stage(1);
    if (!logits) return -1;
    if (plh_forward(&gs.fwd, token, pos, gs.d_fwd_ws, logits, gs.d_x) != 0) {
        backend_lost("plh_forward");
        return -1;
    }
    return forward_done(m, pos, 1);
}

int gpu_try_forward_prefill(model_t *m, const int *tokens, int n_tokens, int start_pos) {
    if (!gpu_available() || !gs.fwd_ready || !same_shape(m) || !tokens) return -1;
    if (n_tokens < 1 || start_pos < 0 || (long)start_pos + n_tokens > (long)gs.max_seq_len)
        return -1;
    for (int i = 0; i < n_tokens; i++)
        if (tokens[i] < 0 || tokens[i] >= m->config.vocab_size) return -1;
    float *logits = forward_stage(n_tokens);
    if (!logits) return -1;
    if (plh_forward_prefill(&gs.fwd, tokens, n_tokens, start_pos, gs.d_fwd_ws, logits,
                            gs.d_x) != 0) {
        backend_lost("plh_forward_prefill");
        return -1;
    }
    return forward_done(m, start_pos, n_tokens);
}
