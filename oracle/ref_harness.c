/*
 * ref_harness.c -- drives the REFERENCE's own forward pass on a tiny
 * in-memory model so that the oracle can be pinned against it.
 *
 * TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile, in this container only,
 * from the sources where they lie under /root/reference/picolm (model.c is
 * included textually because the attention block is inline in
 * model_forward_ex / model_forward_prefill and init_rope_tables and
 * allocate_run_state are static).  Output goes to oracle/_ref/.
 *
 * The model is built so that the attention block's inputs and outputs are
 * observable exactly:
 *   - F32 weights; attn/ffn/output norm weights = 1.
 *   - attn_output (Wo) and output = identity, so s->xb2 after the last layer
 *     holds that layer's attention output bit-for-bit (vec_dot against a unit
 *     row adds only exact zeros), and the logits equal rmsnorm(x_last).
 *   - ffn_gate/up/down = 0, so the FFN adds exact zeros to the residual.
 *   - decode mode: Wq = Wk = Wv = 0 and the per-layer biases carry the chosen
 *     q/k/v exactly (0 + b = b).
 *   - prefill mode: Wq, Wk, Wv random, no biases; ref_layer_inputs recomputes
 *     the layer's q/k/v with the reference's own rmsnorm/matmul_batch calls.
 */
#include "model.c"

#include <stdint.h>

typedef struct {
    model_t m;
    void *blob;
    float *kbias[MAX_LAYERS];
    float *vbias[MAX_LAYERS];
} ref_handle;

static uint64_t hz_state;
static float hz_uniform(void) {
    uint64_t z = (hz_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)((double)(z >> 11) * 0x1p-53 * 2.0 - 1.0);
}

/* mode 0 = decode injection through biases, 1 = prefill with random Wq/Wk/Wv */
void *ref_model_new(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                    int max_seq_len, float rope_base, int rope_type, int mode,
                    unsigned long long seed, float w_scale) {
    if (n_layers < 1 || n_layers > MAX_LAYERS) return NULL;
    ref_handle *h = (ref_handle *)calloc(1, sizeof(ref_handle));
    if (!h) return NULL;
    model_t *m = &h->m;
    model_config_t *c = &m->config;
    int dim = n_heads * head_dim;
    int kv_dim = n_kv_heads * head_dim;
    int n_ffn = 16;
    c->n_embd = dim;
    c->n_ffn = n_ffn;
    c->n_heads = n_heads;
    c->n_kv_heads = n_kv_heads;
    c->n_layers = n_layers;
    c->vocab_size = dim;
    c->max_seq_len = max_seq_len;
    c->head_dim = head_dim;
    c->rope_freq_base = rope_base;
    c->rms_norm_eps = 1e-5f;
    c->rope_type = (rope_type_t)rope_type;
    c->weight_type = GGUF_TYPE_F32;

    size_t per_layer = (size_t)dim * 2                 /* attn_norm, ffn_norm */
                     + (size_t)dim * dim               /* Wq */
                     + (size_t)kv_dim * dim * 2        /* Wk, Wv */
                     + (size_t)dim * dim               /* Wo */
                     + (size_t)n_ffn * dim * 3         /* gate, up, down */
                     + (size_t)kv_dim * 2;             /* k/v bias */
    size_t total = (size_t)dim * dim                   /* token_embd */
                 + (size_t)dim                         /* output_norm */
                 + (size_t)dim * dim                   /* output */
                 + per_layer * (size_t)n_layers;
    float *p = (float *)calloc(total, sizeof(float));
    if (!p) { free(h); return NULL; }
    h->blob = p;
    hz_state = seed;

    float *embd = p; p += (size_t)dim * dim;
    for (size_t i = 0; i < (size_t)dim * dim; i++) embd[i] = hz_uniform();
    float *onorm = p; p += dim;
    for (int i = 0; i < dim; i++) onorm[i] = 1.0f;
    float *wout = p; p += (size_t)dim * dim;
    for (int i = 0; i < dim; i++) wout[(size_t)i * dim + i] = 1.0f;
    m->weights.token_embd = embd;
    m->weights.type_token_embd = GGUF_TYPE_F32;
    m->weights.output_norm = onorm;
    m->weights.type_output_norm = GGUF_TYPE_F32;
    m->weights.output = wout;
    m->weights.type_output = GGUF_TYPE_F32;

    for (int l = 0; l < n_layers; l++) {
        layer_weights_t *lw = &m->weights.layers[l];
        float *an = p; p += dim;
        float *fn = p; p += dim;
        for (int i = 0; i < dim; i++) { an[i] = 1.0f; fn[i] = 1.0f; }
        float *wq = p; p += (size_t)dim * dim;
        float *wk = p; p += (size_t)kv_dim * dim;
        float *wv = p; p += (size_t)kv_dim * dim;
        if (mode == 1) {
            for (size_t i = 0; i < (size_t)dim * dim; i++) wq[i] = hz_uniform() * w_scale;
            for (size_t i = 0; i < (size_t)kv_dim * dim; i++) wk[i] = hz_uniform() * w_scale;
            for (size_t i = 0; i < (size_t)kv_dim * dim; i++) wv[i] = hz_uniform() * w_scale;
        }
        float *wo = p; p += (size_t)dim * dim;
        for (int i = 0; i < dim; i++) wo[(size_t)i * dim + i] = 1.0f;
        float *gate = p; p += (size_t)n_ffn * dim;
        float *up = p; p += (size_t)n_ffn * dim;
        float *down = p; p += (size_t)n_ffn * dim;
        h->kbias[l] = p; p += kv_dim;
        h->vbias[l] = p; p += kv_dim;
        lw->attn_norm = an;
        lw->ffn_norm = fn;
        lw->attn_q = wq;
        lw->attn_k = wk;
        lw->attn_v = wv;
        lw->attn_output = wo;
        lw->ffn_gate = gate;
        lw->ffn_up = up;
        lw->ffn_down = down;
        if (mode == 0) {
            lw->attn_k_b = h->kbias[l];
            lw->attn_v_b = h->vbias[l];
        }
        /* all type_* fields stay GGUF_TYPE_F32 (= 0) from calloc */
    }
    if (allocate_run_state(m) != 0) {
        free(h->blob);
        free(h);
        return NULL;
    }
    return h;
}

/* The reference's own model_t of a handle (run state from allocate_run_state),
 * for harnesses built against picolm's model.h. */
model_t *ref_model(void *hv) { return &((ref_handle *)hv)->m; }

void ref_model_free(void *hv) {
    ref_handle *h = (ref_handle *)hv;
    if (!h) return;
    free(h->m.state.mem_block);
    free(h->m.state.kv_block);
    free(h->blob);
    free(h);
}

void ref_cache_ptrs(void *hv, uint16_t **kc, uint16_t **vc, float **cos_tab,
                    float **sin_tab) {
    ref_handle *h = (ref_handle *)hv;
    *kc = h->m.state.key_cache;
    *vc = h->m.state.val_cache;
    *cos_tab = h->m.state.rope_cos;
    *sin_tab = h->m.state.rope_sin;
}

/* Decode mode: the q/k/v that layer `layer` will see (exact, via biases). */
void ref_set_decode_qkv(void *hv, int layer, const float *q, const float *k,
                        const float *v) {
    ref_handle *h = (ref_handle *)hv;
    model_config_t *c = &h->m.config;
    int q_dim = c->n_heads * c->head_dim;
    int kv_dim = c->n_kv_heads * c->head_dim;
    memcpy(h->m.state.attn_q_bias[layer], q, (size_t)q_dim * sizeof(float));
    memcpy(h->kbias[layer], k, (size_t)kv_dim * sizeof(float));
    memcpy(h->vbias[layer], v, (size_t)kv_dim * sizeof(float));
}

/* Runs the reference's model_forward_ex for layers [0, n_layers_run) at
 * position pos and returns the attention output of the last layer run. */
void ref_decode(void *hv, int pos, int n_layers_run, float *attn_out) {
    ref_handle *h = (ref_handle *)hv;
    model_forward_ex(&h->m, 0, pos, n_layers_run);
    memcpy(attn_out, h->m.state.xb2, (size_t)h->m.config.n_embd * sizeof(float));
}

/* Runs the reference's model_forward_prefill; returns the last token's logits
 * (= rmsnorm(x_last) with unit weights, since the output matrix is I). */
void ref_prefill(void *hv, const int *tokens, int n_tokens, int start_pos,
                 float *logits) {
    ref_handle *h = (ref_handle *)hv;
    model_forward_prefill(&h->m, tokens, n_tokens, start_pos);
    memcpy(logits, h->m.state.logits, (size_t)h->m.config.vocab_size * sizeof(float));
}

/* Embedding rows as model_forward_prefill reads them (model.c:977-982). */
void ref_embed(void *hv, const int *tokens, int n_tokens, float *x) {
    ref_handle *h = (ref_handle *)hv;
    int dim = h->m.config.n_embd;
    for (int bi = 0; bi < n_tokens; bi++) {
        const float *row = (const float *)h->m.weights.token_embd + (size_t)tokens[bi] * dim;
        dequantize_row(row, x + (size_t)bi * dim, dim, GGUF_TYPE_F32);
    }
}

/* The q/k/v model_forward_prefill computes for layer `layer` from the
 * residual stream x (model.c:988-1000), with the same function calls. */
void ref_layer_inputs(void *hv, int layer, const float *x, int n_tokens,
                      float *q, float *k, float *v) {
    ref_handle *h = (ref_handle *)hv;
    model_config_t *c = &h->m.config;
    layer_weights_t *lw = &h->m.weights.layers[layer];
    int dim = c->n_embd;
    int q_dim = c->n_heads * c->head_dim;
    int kv_dim = c->n_kv_heads * c->head_dim;
    float *xb = (float *)malloc((size_t)n_tokens * dim * sizeof(float));
    for (int bi = 0; bi < n_tokens; bi++)
        rmsnorm(xb + (size_t)bi * dim, x + (size_t)bi * dim,
                h->m.state.attn_norm_w[layer], dim, c->rms_norm_eps);
    matmul_batch(q, xb, n_tokens, lw->attn_q, dim, q_dim, lw->type_attn_q);
    matmul_dual_batch(k, v, xb, n_tokens, lw->attn_k, lw->attn_v, dim, kv_dim,
                      lw->type_attn_k, lw->type_attn_v);
    free(xb);
}

/* Final norm as model_forward_prefill applies it to the last token. */
void ref_final_norm(void *hv, const float *x, float *out) {
    ref_handle *h = (ref_handle *)hv;
    rmsnorm(out, x, h->m.state.output_norm_w, h->m.config.n_embd,
            h->m.config.rms_norm_eps);
}

/* Exhaustive comparison of the reference's fp32_to_fp16 (quant.c:41-78)
 * against another implementation over fp32 bit patterns [first, first+count).
 * Returns the number of mismatching inputs; *first_bad gets the lowest one. */
#include <pthread.h>

typedef uint16_t (*f2h_fn)(float);
typedef struct {
    uint64_t first, count, bad;
    uint32_t first_bad;
    f2h_fn other;
} cmp_job;

static void *cmp_worker(void *arg) {
    cmp_job *j = (cmp_job *)arg;
    j->bad = 0;
    j->first_bad = 0xFFFFFFFFu;
    for (uint64_t i = 0; i < j->count; i++) {
        uint32_t bits = (uint32_t)(j->first + i);
        float f;
        memcpy(&f, &bits, sizeof f);
        if (fp32_to_fp16(f) != j->other(f)) {
            if (j->bad == 0) j->first_bad = bits;
            j->bad++;
        }
    }
    return NULL;
}

uint64_t ref_f16_mismatches(uint64_t first, uint64_t count, f2h_fn other,
                            int n_threads, uint32_t *first_bad) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    cmp_job jobs[64];
    uint64_t per = count / (uint64_t)n_threads, at = first;
    for (int t = 0; t < n_threads; t++) {
        jobs[t].first = at;
        jobs[t].count = (t == n_threads - 1) ? first + count - at : per;
        jobs[t].other = other;
        at += jobs[t].count;
    }
    for (int t = 1; t < n_threads; t++) pthread_create(&th[t], NULL, cmp_worker, &jobs[t]);
    cmp_worker(&jobs[0]);
    uint64_t bad = jobs[0].bad;
    uint32_t fb = jobs[0].first_bad;
    for (int t = 1; t < n_threads; t++) {
        pthread_join(th[t], NULL);
        bad += jobs[t].bad;
        if (jobs[t].bad && (fb == 0xFFFFFFFFu)) fb = jobs[t].first_bad;
    }
    *first_bad = fb;
    return bad;
}

/* The reference's fp16_to_fp32 (quant.c:11-39) over an array, bits kept
 * in C so that signalling NaN payloads are not quieted by a host-language
 * float conversion. */
void ref_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = fp16_to_fp32(src[i]);
}

/* Qwen3 QK-norm for layer `layer` (model.c:807-817, 1029-1037): the layer's
 * attn_q_norm / attn_k_norm tensors become non-null and the run state's
 * dequantised per-head weights (model.c:657-670) take q_w / k_w; eps becomes
 * the model's rms_norm_eps. */
void ref_set_qk_norm(void *hv, int layer, const float *q_w, const float *k_w, float eps) {
    ref_handle *h = (ref_handle *)hv;
    model_t *m = &h->m;
    int D = m->config.head_dim;
    memcpy(m->state.attn_q_norm_w[layer], q_w, (size_t)D * sizeof(float));
    memcpy(m->state.attn_k_norm_w[layer], k_w, (size_t)D * sizeof(float));
    m->weights.layers[layer].attn_q_norm = m->state.attn_q_norm_w[layer];
    m->weights.layers[layer].attn_k_norm = m->state.attn_k_norm_w[layer];
    m->weights.layers[layer].type_attn_q_norm = GGUF_TYPE_F32;
    m->weights.layers[layer].type_attn_k_norm = GGUF_TYPE_F32;
    m->config.rms_norm_eps = eps;
}

/* The reference's rmsnorm (tensor.c:425-492) as this harness is built. */
void ref_rmsnorm(float *out, const float *x, const float *w, int size, float eps) {
    rmsnorm(out, x, w, size, eps);
}

/* A model assembled from caller-owned buffers, for pinning the oracle's
 * whole forward pass against model_forward / model_forward_prefill.
 * cfg = {n_layers, n_embd, n_ffn, n_heads, n_kv_heads, head_dim, vocab_size,
 * max_seq_len, rope_type}.  ptrs/types hold, in this order, token_embd,
 * output_norm, output, then per layer attn_norm, attn_q, attn_k, attn_v,
 * attn_output, attn_q_norm, attn_k_norm, ffn_norm, ffn_gate, ffn_down,
 * ffn_up, attn_q_b, attn_k_b, attn_v_b, attn_output_b (NULL = absent).
 * allocate_run_state then dequantizes norms and biases and builds the RoPE
 * tables exactly as model_load does (model.c:721-730). */
#define REF_LAYER_SLOTS 15
void *ref_model_new_full(const int *cfg, float rope_base, float eps, const void *const *ptrs,
                         const int *types) {
    if (cfg[0] < 1 || cfg[0] > MAX_LAYERS) return NULL;
    ref_handle *h = (ref_handle *)calloc(1, sizeof(ref_handle));
    if (!h) return NULL;
    model_t *m = &h->m;
    model_config_t *c = &m->config;
    c->n_layers = cfg[0];
    c->n_embd = cfg[1];
    c->n_ffn = cfg[2];
    c->n_heads = cfg[3];
    c->n_kv_heads = cfg[4];
    c->head_dim = cfg[5];
    c->vocab_size = cfg[6];
    c->max_seq_len = cfg[7];
    c->rope_type = (rope_type_t)cfg[8];
    c->rope_freq_base = rope_base;
    c->rms_norm_eps = eps;
    c->weight_type = GGUF_TYPE_F32;
    model_weights_t *w = &m->weights;
    w->token_embd = ptrs[0];
    w->type_token_embd = (gguf_type_t)types[0];
    w->output_norm = ptrs[1];
    w->type_output_norm = (gguf_type_t)types[1];
    w->output = ptrs[2];
    w->type_output = (gguf_type_t)types[2];
    for (int l = 0; l < c->n_layers; l++) {
        const void *const *p = ptrs + 3 + (size_t)l * REF_LAYER_SLOTS;
        const int *t = types + 3 + (size_t)l * REF_LAYER_SLOTS;
        layer_weights_t *lw = &w->layers[l];
        lw->attn_norm = p[0];     lw->type_attn_norm = (gguf_type_t)t[0];
        lw->attn_q = p[1];        lw->type_attn_q = (gguf_type_t)t[1];
        lw->attn_k = p[2];        lw->type_attn_k = (gguf_type_t)t[2];
        lw->attn_v = p[3];        lw->type_attn_v = (gguf_type_t)t[3];
        lw->attn_output = p[4];   lw->type_attn_output = (gguf_type_t)t[4];
        lw->attn_q_norm = p[5];   lw->type_attn_q_norm = (gguf_type_t)t[5];
        lw->attn_k_norm = p[6];   lw->type_attn_k_norm = (gguf_type_t)t[6];
        lw->ffn_norm = p[7];      lw->type_ffn_norm = (gguf_type_t)t[7];
        lw->ffn_gate = p[8];      lw->type_ffn_gate = (gguf_type_t)t[8];
        lw->ffn_down = p[9];      lw->type_ffn_down = (gguf_type_t)t[9];
        lw->ffn_up = p[10];       lw->type_ffn_up = (gguf_type_t)t[10];
        lw->attn_q_b = p[11];     lw->type_attn_q_b = (gguf_type_t)t[11];
        lw->attn_k_b = p[12];     lw->type_attn_k_b = (gguf_type_t)t[12];
        lw->attn_v_b = p[13];     lw->type_attn_v_b = (gguf_type_t)t[13];
        lw->attn_output_b = p[14]; lw->type_attn_output_b = (gguf_type_t)t[14];
    }
    if (allocate_run_state(m) != 0) {
        free(h);
        return NULL;
    }
    return h;
}

/* model_forward (model.c:742-744): logits and the final normalised residual. */
void ref_forward(void *hv, int token, int pos, float *logits, float *x_out) {
    ref_handle *h = (ref_handle *)hv;
    float *lg = model_forward(&h->m, token, pos);
    memcpy(logits, lg, (size_t)h->m.config.vocab_size * sizeof(float));
    memcpy(x_out, h->m.state.x, (size_t)h->m.config.n_embd * sizeof(float));
}

/* model_forward_prefill (model.c:939-1144). */
void ref_forward_prefill(void *hv, const int *tokens, int n_tokens, int start_pos,
                         float *logits, float *x_out) {
    ref_handle *h = (ref_handle *)hv;
    model_forward_prefill(&h->m, tokens, n_tokens, start_pos);
    memcpy(logits, h->m.state.logits, (size_t)h->m.config.vocab_size * sizeof(float));
    memcpy(x_out, h->m.state.x, (size_t)h->m.config.n_embd * sizeof(float));
}

/* tensor.c:605-609 over an array (silu in place). */
void ref_silu(float *x, int n) { silu(x, n); }

/* tensor.c:190-195: the matmul thread-pool size of every later call. */
void ref_set_threads(int n) { tensor_set_threads(n); }
