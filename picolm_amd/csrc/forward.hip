// forward.hip -- picolm's forward pass for one token (model_forward_ex,
// model.c:746-925) on the device, around the attention and GEMV kernels:
// embedding row dequantisation, rmsnorm, the projections with their bias /
// SwiGLU / residual epilogues, attention, the final norm and the logits.
//
// Every step but two is bit-identical to the reference's x86-64 build: the
// embedding (quant.c:96-128, 193-262), rmsnorm (tensor.c:425-492, AVX2
// order), the GEMVs, biases and residual adds (tensor.c:200-264, 635-657).
// The two that are not: silu's expf (the device library's, where glibc's
// expf is not correctly rounded either) and the attention softmax (split
// over positions, exp2-based); both stay within a few ulps per value.
#include <stdint.h>

#include "attn_common.h"
#include "picolm_hip.h"
#include "plh_internal.h"

using namespace plh;

namespace plh {
int g_fwd_norm_separate = 0;
}

namespace {

constexpr int kTypeF32 = 0, kTypeF16 = 1, kTypeQ4_0 = 2, kTypeQ8_0 = 8, kTypeQ4K = 12,
              kTypeQ6K = 14;
constexpr int kNormThreads = 256;
constexpr int kMaxNormSize = 12288;  // the squares of a row must fit 48 KiB of LDS

// ---- rmsnorm (tensor.c:425-492, x86-64 AVX2 path) --------------------------
// One workgroup: the reference's scale (rms_scale_block), then
// out[i] = (x[i] * scale) * w[i].  Device division and square root are
// correctly rounded, so the output is the reference's bit for bit.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* x, const float* w,
                                                               float* out, int n, float eps) {
  extern __shared__ __align__(16) float sq[];
  __shared__ float red[8];
  const float scale = rms_scale_block<kNormThreads>(x, n, eps, sq, red);
  for (int i = threadIdx.x; i < n; i += kNormThreads) {
    const float t = x[i] * scale;
    out[i] = t * w[i];
  }
}

// rmsnorm of n_rows rows (one workgroup each), rows `stride` floats apart.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_rows_kernel(const float* x,
                                                                    const float* w, float* out,
                                                                    int n, int stride, float eps) {
  extern __shared__ __align__(16) float sq[];
  __shared__ float red[8];
  const float* xr = x + (size_t)blockIdx.x * stride;
  float* orow = out + (size_t)blockIdx.x * stride;
  const float scale = rms_scale_block<kNormThreads>(xr, n, eps, sq, red);
  for (int i = threadIdx.x; i < n; i += kNormThreads) {
    const float t = xr[i] * scale;
    orow[i] = t * w[i];
  }
}

// ---- one GGUF row to fp32 (quant.c:96-128, 193-262) ------------------------
__device__ __forceinline__ uint32_t rd8(const uint8_t* p) { return p[0]; }
__device__ __forceinline__ uint16_t rd16(const uint8_t* p) {
  return (uint16_t)(p[0] | (p[1] << 8));
}

// get_scale_min_k4 (quant.c:82-91)
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t* q, int& sc, int& mn) {
  if (j < 4) {
    sc = q[j] & 63;
    mn = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// Element e of a GGUF row.
__device__ __forceinline__ float dequant_elem(int qtype, const uint8_t* row, int e) {
  float y = 0.0f;
  switch (qtype) {
    case kTypeF32: {
      const uint8_t* p = row + 4 * (size_t)e;
      y = __uint_as_float(p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24));
      break;
    }
    case kTypeF16:
      y = f16_bits_to_f32(rd16(row + 2 * (size_t)e));
      break;
    case kTypeQ4_0: {  // {fp16 d, qs[16]}: element j < 16 low nibble of qs[j], else high of qs[j-16]
      const uint8_t* b = row + (size_t)(e / 32) * 18;
      const int j = e % 32;
      const int nib = j < 16 ? (b[2 + j] & 0xF) : (b[2 + j - 16] >> 4);
      y = f16_bits_to_f32(rd16(b)) * ((float)nib - 8.0f);
      break;
    }
    case kTypeQ8_0: {
      const uint8_t* b = row + (size_t)(e / 32) * 34;
      y = f16_bits_to_f32(rd16(b)) * (float)(int8_t)rd8(b + 2 + e % 32);
      break;
    }
    case kTypeQ4K: {  // {fp16 d, fp16 dmin, scales[12], qs[128]}
      const uint8_t* b = row + (size_t)(e / 256) * 144;
      const int r = e % 256, j = r / 64, hi = (r % 64) >= 32, l = r % 32;
      int sc, mn;
      q4k_scale_min(2 * j + hi, b + 4, sc, mn);
      const float d1 = f16_bits_to_f32(rd16(b)) * (float)sc;
      const float m1 = f16_bits_to_f32(rd16(b + 2)) * (float)mn;
      const int q = b[16 + 32 * j + l];
      const float a = d1 * (float)(hi ? (q >> 4) : (q & 0xF));
      y = a - m1;
      break;
    }
    case kTypeQ6K: {  // {ql[128], qh[64], int8 scales[16], fp16 d}
      const uint8_t* b = row + (size_t)(e / 256) * 210;
      const int r = e % 256, c = r / 128, quarter = (r % 128) / 32, l = r % 32;
      const int lo = b[64 * c + l + ((quarter & 1) ? 32 : 0)];
      const int nib = (quarter & 2) ? (lo >> 4) : (lo & 0xF);
      const int q = (nib | (((b[128 + 32 * c + l] >> (2 * quarter)) & 3) << 4)) - 32;
      const float ds = f16_bits_to_f32(rd16(b + 208)) * (float)(int8_t)b[192 + r / 16];
      y = ds * (float)q;
      break;
    }
    default:
      break;
  }
  return y;
}

__global__ __launch_bounds__(256) void dequant_row_kernel(int qtype, const uint8_t* row,
                                                          float* out, int n) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e < n) out[e] = dequant_elem(qtype, row, e);
}

// The embedding rows of up to kEmbedTokens tokens (model.c:976-982), one
// workgroup row per token, rows `stride` floats apart.
constexpr int kEmbedTokens = 64;
struct EmbedArgs {
  int tokens[kEmbedTokens];
  int n_tok, qtype, n, stride;
  size_t row_bytes;
  const uint8_t* table;
  float* x;
};
__global__ __launch_bounds__(256) void embed_rows_kernel(EmbedArgs a) {
  const int t = blockIdx.y;
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (t >= a.n_tok || e >= a.n) return;
  a.x[(size_t)t * a.stride + e] =
      dequant_elem(a.qtype, a.table + (size_t)a.tokens[t] * a.row_bytes, e);
}

size_t embd_row_bytes(int qtype, int n) {
  switch (qtype) {
    case kTypeF32: return (size_t)n * 4;
    case kTypeF16: return (size_t)n * 2;
    case kTypeQ4_0: return n % 32 ? 0 : (size_t)(n / 32) * 18;
    case kTypeQ8_0: return n % 32 ? 0 : (size_t)(n / 32) * 34;
    case kTypeQ4K: return n % 256 ? 0 : (size_t)(n / 256) * 144;
    case kTypeQ6K: return n % 256 ? 0 : (size_t)(n / 256) * 210;
    default: return 0;
  }
}

size_t norm_lds_bytes(int n) { return sizeof(float) * 8 * (size_t)rms_sq_pitch(n); }

int launch_rmsnorm(const float* x, const float* w, float* out, int n, float eps) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(kNormThreads), norm_lds_bytes(n), ctx().stream,
                     x, w, out, n, eps);
  return check_hip(hipGetLastError(), "rmsnorm_kernel launch");
}

// Workspace carve-up of plh_forward, 256-byte aligned pieces.
struct Acts {
  float *x, *xb, *q, *k, *v, *att, *hb;
  size_t bytes;
};

size_t piece(size_t floats) { return (floats * sizeof(float) + 255) / 256 * 256; }

Acts carve(const plh_model* m, void* base) {
  const size_t q_dim = (size_t)m->n_heads * m->head_dim;
  const size_t kv_dim = (size_t)m->n_kv_heads * m->head_dim;
  const size_t sizes[7] = {(size_t)m->n_embd, (size_t)m->n_embd, q_dim, kv_dim, kv_dim, q_dim,
                           (size_t)m->n_ffn};
  Acts a{};
  float** dst[7] = {&a.x, &a.xb, &a.q, &a.k, &a.v, &a.att, &a.hb};
  size_t off = 0;
  for (int i = 0; i < 7; ++i) {
    *dst[i] = base ? (float*)((char*)base + off) : nullptr;
    off += piece(sizes[i]);
  }
  a.bytes = off;
  return a;
}

bool gemv_type(int qtype) { return qtype == kTypeQ4K || qtype == kTypeQ6K || qtype == kTypeQ8_0; }

bool matrix_ok(const plh_matrix& w, int n, int d) {
  return w.w && gemv_type(w.qtype) && plh_gemv_packed_bytes(w.qtype, n, d) > 0;
}

// Checks everything plh_forward relies on; sets the error and returns false
// otherwise.
bool model_ok(const plh_model* m) {
  if (!m || !m->layers) {
    set_error("plh_forward: null model or layer table");
    return false;
  }
  if (m->n_layers < 1 || m->n_embd < 1 || m->n_ffn < 1 || m->vocab_size < 1 ||
      m->max_seq_len < 1 || m->n_heads < 1 || m->n_kv_heads < 1 ||
      m->n_heads % m->n_kv_heads || m->head_dim < 2 || m->head_dim > 256 || m->head_dim % 2 ||
      (m->rope_type != PLH_ROPE_LLAMA && m->rope_type != PLH_ROPE_QWEN)) {
    set_error("plh_forward: unsupported shape (layers %d, embd %d, heads %d/%d, head_dim %d)",
              m->n_layers, m->n_embd, m->n_heads, m->n_kv_heads, m->head_dim);
    return false;
  }
  if (m->n_embd > kMaxNormSize) {
    set_error("plh_forward: n_embd %d exceeds %d", m->n_embd, kMaxNormSize);
    return false;
  }
  const int q_dim = m->n_heads * m->head_dim, kv_dim = m->n_kv_heads * m->head_dim;
  if (!m->token_embd || embd_row_bytes(m->embd_type, m->n_embd) == 0) {
    set_error("plh_forward: no device dequantisation for embedding type %d", m->embd_type);
    return false;
  }
  if (!m->output_norm || !m->key_cache || !m->val_cache || !m->rope_cos || !m->rope_sin ||
      !matrix_ok(m->output, m->n_embd, m->vocab_size)) {
    set_error("plh_forward: missing output norm / output matrix / caches / tables");
    return false;
  }
  for (int l = 0; l < m->n_layers; ++l) {
    const plh_layer& L = m->layers[l];
    if (!L.attn_norm || !L.ffn_norm || !matrix_ok(L.q, m->n_embd, q_dim) ||
        !matrix_ok(L.k, m->n_embd, kv_dim) || !matrix_ok(L.v, m->n_embd, kv_dim) ||
        !matrix_ok(L.o, q_dim, m->n_embd) || !matrix_ok(L.gate, m->n_embd, m->n_ffn) ||
        !matrix_ok(L.up, m->n_embd, m->n_ffn) || !matrix_ok(L.down, m->n_ffn, m->n_embd)) {
      set_error("plh_forward: layer %d lacks a norm or a GEMV-capable matrix", l);
      return false;
    }
    if ((L.q_norm == nullptr) != (L.k_norm == nullptr)) {
      set_error("plh_forward: layer %d has only one of q_norm / k_norm", l);
      return false;
    }
  }
  return true;
}

}  // namespace

extern "C" {

int plh_rmsnorm(const float* x, const float* w, float* out, int n, float eps) {
  if (!ctx().stream) {
    set_error("plh_rmsnorm: plh_init has not been called");
    return -1;
  }
  if (!x || !w || !out || n < 1 || n > kMaxNormSize) {
    set_error("plh_rmsnorm: bad arguments (n = %d, at most %d)", n, kMaxNormSize);
    return -1;
  }
  return launch_rmsnorm(x, w, out, n, eps);
}

int plh_dequantize_row(int qtype, const void* row, float* out, int n) {
  if (!ctx().stream) {
    set_error("plh_dequantize_row: plh_init has not been called");
    return -1;
  }
  if (!row || !out || n < 1 || embd_row_bytes(qtype, n) == 0) {
    set_error("plh_dequantize_row: no row of %d weights of type %d", n, qtype);
    return -1;
  }
  hipLaunchKernelGGL(dequant_row_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx().stream, qtype,
                     (const uint8_t*)row, out, n);
  return check_hip(hipGetLastError(), "dequant_row_kernel launch");
}

size_t plh_forward_workspace_bytes(const plh_model* m) {
  if (!m) return 0;
  return carve(m, nullptr).bytes;
}

}  // extern "C"

namespace {

// One token through every layer, the final norm and the logits (arguments
// checked by the caller).  The q and output biases follow model_forward_ex:
// added always, zeros when absent (model.c:781-782 / 895-896), which turns a
// -0 sum into +0 where model_forward_prefill, adding only present biases,
// would not.
int forward_token(const plh_model* m, int token, int pos, void* workspace, float* logits,
                  float* x_out) {
  const int E = m->n_embd, F = m->n_ffn;
  const int Q = m->n_heads * m->head_dim, KV = m->n_kv_heads * m->head_dim;
  const float eps = m->rms_norm_eps;
  const Acts a = carve(m, workspace);
  const size_t rb = embd_row_bytes(m->embd_type, E);
  if (plh_dequantize_row(m->embd_type, (const uint8_t*)m->token_embd + (size_t)token * rb, a.x,
                         E))
    return -1;
  // every GEMV that reads rmsnorm(x) forms it itself (tensor.c:425-492)
  auto call = [&](const plh_matrix& w, int n, int d, const float* x, float* out,
                  const float* norm_w, const float* bias, int bias_zero, const float* gate,
                  const float* resid) {
    GemvCall g{};
    g.qtype = w.qtype, g.n = n, g.d = d, g.w = w.w, g.x = x, g.out = out;
    g.norm_w = norm_w, g.norm_eps = eps;
    g.bias = bias, g.bias_zero = bias_zero, g.gate = gate, g.resid = resid;
    return g;
  };
  // rmsnorm(x, w): inside the GEMVs that read it, or (tuning key 4) one
  // launch of its own into xb; returns the GEMV operand and its prologue
  const bool separate = g_fwd_norm_separate != 0 || E > kGemvNormMax;
  auto normed = [&](const float* w, const float** xin, const float** nw) {
    *xin = separate ? a.xb : a.x;
    *nw = separate ? nullptr : w;
    return separate ? launch_rmsnorm(a.x, w, a.xb, E, eps) : 0;
  };
  const float *xin, *nw;
  for (int l = 0; l < m->n_layers; ++l) {
    const plh_layer& L = m->layers[l];
    // attention block (model.c:777-897): q, k, v in one launch
    if (normed(L.attn_norm, &xin, &nw)) return -1;
    const GemvCall qkv[3] = {
        call(L.q, E, Q, xin, a.q, nw, L.q_bias, !L.q_bias, nullptr, nullptr),
        call(L.k, E, KV, xin, a.k, nw, L.k_bias, 0, nullptr, nullptr),
        call(L.v, E, KV, xin, a.v, nw, L.v_bias, 0, nullptr, nullptr)};
    // At short context q, k, v and the attention run in one launch (tuning
    // key 17): the attention workgroups wait for their group's rows instead
    // of a launch boundary (qkv_attention_launch).
    DecodeArgs fd;
    unsigned* fctr = nullptr;
    const bool fuse = g_fwd_fuse >= 0 && !L.q_norm && nw != nullptr && !g_gemv_exact &&
                      decode_args_fused(m->n_layers, m->n_heads, m->n_kv_heads, m->head_dim,
                                        m->max_seq_len, m->rope_type, l, pos, a.q, a.k, a.v,
                                        m->key_cache, m->val_cache, m->rope_cos, m->rope_sin,
                                        a.att, fd, &fctr);
    if (!fuse && gemv_multi_launch(qkv, 3)) return -1;
    // The attention launch (or the fused one) leaves most CUs idle: extra
    // workgroups bring the o-projection's, the gate/up pair's and the down
    // projection's weights into the L2 of the XCDs whose GEMV workgroups will
    // read them.
    PfPlan& pf = ctx().pf_next;
    pf.n = 0;
    if (g_fwd_prefetch >= 0) {
      const float* ffn_nw = separate ? nullptr : L.ffn_norm;
      const float* ffn_x = separate ? a.xb : a.x;
      const GemvCall o = call(L.o, Q, E, a.att, a.x, nullptr, L.o_bias, !L.o_bias, nullptr, a.x);
      const GemvCall g = call(L.gate, E, F, ffn_x, a.hb, ffn_nw, nullptr, 0, nullptr, nullptr);
      const GemvCall u = call(L.up, E, F, ffn_x, a.hb, ffn_nw, nullptr, 0, nullptr, nullptr);
      gemv_prefetch_plan(o, nullptr, pf);
      if (L.gate.qtype == L.up.qtype) gemv_prefetch_plan(g, &u, pf);
      if (g_fwd_prefetch == 0)
        gemv_prefetch_plan(call(L.down, F, E, a.hb, a.x, nullptr, nullptr, 0, nullptr, a.x),
                           nullptr, pf);
    }
    int rc;
    if (fuse)
      rc = qkv_attention_launch(qkv, fd, m->head_dim, fctr, pf,
                                g_fwd_fuse >= 8 ? g_fwd_fuse : kFusePrefetchPerXcd);
    else if (L.q_norm)
      rc = plh_attn_decode_qknorm(m->n_layers, m->n_heads, m->n_kv_heads, m->head_dim,
                                  m->max_seq_len, m->rope_type, l, 1, pos, a.q, a.k, a.v,
                                  m->key_cache, m->val_cache, m->rope_cos, m->rope_sin, a.att,
                                  L.q_norm, L.k_norm, eps);
    else
      rc = plh_attn_decode(m->n_layers, m->n_heads, m->n_kv_heads, m->head_dim,
                           m->max_seq_len, m->rope_type, l, 1, pos, a.q, a.k, a.v, m->key_cache,
                           m->val_cache, m->rope_cos, m->rope_sin, a.att);
    pf.n = 0;
    if (rc) return -1;
    // x = x + (Wo att + o_bias)
    if (gemv_launch(call(L.o, Q, E, a.att, a.x, nullptr, L.o_bias, !L.o_bias, nullptr, a.x)))
      return -1;
    // SwiGLU block (model.c:899-922): hb = silu(gate xn) * (up xn), xn = rmsnorm(x),
    // in one launch when gate and up share a type; then x = x + Wdown hb
    if (normed(L.ffn_norm, &xin, &nw)) return -1;
    const GemvCall gate = call(L.gate, E, F, xin, a.hb, nw, nullptr, 0, nullptr, nullptr);
    const GemvCall up = call(L.up, E, F, xin, a.hb, nw, nullptr, 0, nullptr, nullptr);
    if (L.gate.qtype == L.up.qtype) {
      if (gemv_pair_launch(gate, up)) return -1;
    } else {
      GemvCall up_g = up;
      up_g.gate = a.hb;
      if (gemv_launch(gate) || gemv_launch(up_g)) return -1;
    }
    if (gemv_launch(call(L.down, F, E, a.hb, a.x, nullptr, nullptr, 0, nullptr, a.x))) return -1;
  }
  // final norm and logits (model.c:918-922)
  if (normed(m->output_norm, &xin, &nw)) return -1;
  GemvCall out = call(m->output, E, m->vocab_size, xin, logits, nw, nullptr, 0, nullptr, nullptr);
  out.xn_out = nw ? x_out : nullptr;  // the prologue's rmsnorm(x) is state.x
  if (gemv_launch(out)) return -1;
  if (x_out && !nw && plh_memcpy_dtod(x_out, xin, (size_t)E * sizeof(float))) return -1;
  return 0;
}


// ---- prompt chunks (model_forward_prefill, model.c:939-1144) ---------------
// A chunk of up to kPrefillChunk prompt tokens goes through each layer
// together: the batched GEMVs (matmul_batch) read every weight about once per
// chunk, the prefill attention kernel appends and attends the chunk's rows.
constexpr int kPrefillChunk = 128;

struct ChunkActs {
  float *x, *xn, *q, *k, *v, *att, *hb;
  size_t bytes;
};

ChunkActs carve_chunk(const plh_model* m, int T, void* base) {
  const size_t q_dim = (size_t)m->n_heads * m->head_dim;
  const size_t kv_dim = (size_t)m->n_kv_heads * m->head_dim;
  const size_t E = (size_t)m->n_embd, F = (size_t)m->n_ffn;
  const size_t sizes[7] = {T * E, T * E, T * q_dim, T * kv_dim, T * kv_dim, T * q_dim, T * F};
  ChunkActs a{};
  float** dst[7] = {&a.x, &a.xn, &a.q, &a.k, &a.v, &a.att, &a.hb};
  size_t off = 0;
  for (int i = 0; i < 7; ++i) {
    *dst[i] = base ? (float*)((char*)base + off) : nullptr;
    off += piece(sizes[i]);
  }
  a.bytes = off;
  return a;
}

int ensure_prefill_ws(size_t bytes) {
  Context& c = ctx();
  if (c.pf_ws && c.pf_ws_bytes >= bytes) return 0;
  return grow_buffer(&c.pf_ws, &c.pf_ws_bytes, bytes + bytes / 2, "hipMalloc(prefill workspace)");
}

int launch_rmsnorm_rows(const float* x, const float* w, float* out, int n, int rows, float eps) {
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(kNormThreads), norm_lds_bytes(n),
                     ctx().stream, x, w, out, n, n, eps);
  return check_hip(hipGetLastError(), "rmsnorm_rows_kernel launch");
}

// Tokens [0, T) of the chunk at positions pos0.. through every layer; on
// return a.x holds their residual streams.
int prefill_chunk(const plh_model* m, const int* tokens, int T, int pos0, const ChunkActs& a) {
  const int E = m->n_embd, F = m->n_ffn;
  const int Q = m->n_heads * m->head_dim, KV = m->n_kv_heads * m->head_dim;
  const float eps = m->rms_norm_eps;
  const size_t rb = embd_row_bytes(m->embd_type, E);
  for (int t0 = 0; t0 < T; t0 += kEmbedTokens) {
    EmbedArgs ea{};
    ea.n_tok = min(kEmbedTokens, T - t0);
    for (int i = 0; i < ea.n_tok; ++i) ea.tokens[i] = tokens[t0 + i];
    ea.qtype = m->embd_type, ea.n = E, ea.stride = E, ea.row_bytes = rb;
    ea.table = (const uint8_t*)m->token_embd;
    ea.x = a.x + (size_t)t0 * E;
    hipLaunchKernelGGL(embed_rows_kernel, dim3((E + 255) / 256, ea.n_tok), dim3(256), 0,
                       ctx().stream, ea);
    if (check_hip(hipGetLastError(), "embed_rows_kernel launch")) return -1;
  }
  auto call = [&](const plh_matrix& w, int n, int d, const float* x, int x_stride, float* out,
                  int out_stride, const float* bias, const float* gate, const float* resid) {
    GemvCall g{};
    g.qtype = w.qtype, g.n = n, g.d = d, g.w = w.w, g.x = x, g.out = out;
    g.bias = bias, g.gate = gate, g.resid = resid;
    g.n_tok = T, g.x_stride = x_stride, g.out_stride = out_stride;
    return g;
  };
  for (int l = 0; l < m->n_layers; ++l) {
    const plh_layer& L = m->layers[l];
    // model.c:988-1017: rmsnorm, q / k / v projections, biases where present
    if (launch_rmsnorm_rows(a.x, L.attn_norm, a.xn, E, T, eps) ||
        gemv_launch(call(L.q, E, Q, a.xn, E, a.q, Q, L.q_bias, nullptr, nullptr)) ||
        gemv_launch(call(L.k, E, KV, a.xn, E, a.k, KV, L.k_bias, nullptr, nullptr)) ||
        gemv_launch(call(L.v, E, KV, a.xn, E, a.v, KV, L.v_bias, nullptr, nullptr)))
      return -1;
    // model.c:1019-1090: QK-norm, RoPE, fp16 append and attention per token
    const int rc =
        L.q_norm ? plh_attn_prefill_qknorm(m->n_layers, m->n_heads, m->n_kv_heads, m->head_dim,
                                           m->max_seq_len, m->rope_type, l, 1, pos0, T, a.q, a.k,
                                           a.v, m->key_cache, m->val_cache, m->rope_cos,
                                           m->rope_sin, a.att, Q, L.q_norm, L.k_norm, eps)
                 : plh_attn_prefill(m->n_layers, m->n_heads, m->n_kv_heads, m->head_dim,
                                    m->max_seq_len, m->rope_type, l, 1, pos0, T, a.q, a.k, a.v,
                                    m->key_cache, m->val_cache, m->rope_cos, m->rope_sin, a.att,
                                    Q);
    if (rc) return -1;
    // model.c:1092-1107: output projection, its bias where present, residual
    if (gemv_launch(call(L.o, Q, E, a.att, Q, a.x, E, L.o_bias, nullptr, a.x))) return -1;
    // model.c:1109-1139: rmsnorm, gate / up, silu * up, down, residual
    if (launch_rmsnorm_rows(a.x, L.ffn_norm, a.xn, E, T, eps)) return -1;
    const GemvCall gate = call(L.gate, E, F, a.xn, E, a.hb, F, nullptr, nullptr, nullptr);
    const GemvCall up = call(L.up, E, F, a.xn, E, a.hb, F, nullptr, nullptr, nullptr);
    if (L.gate.qtype == L.up.qtype) {
      if (gemv_pair_launch(gate, up)) return -1;
    } else {
      GemvCall up_g = up;
      up_g.gate = a.hb;
      if (gemv_launch(gate) || gemv_launch(up_g)) return -1;
    }
    if (gemv_launch(call(L.down, F, E, a.hb, F, a.x, E, nullptr, nullptr, a.x))) return -1;
  }
  return 0;
}

}  // namespace

extern "C" {

int plh_forward(const plh_model* m, int token, int pos, void* workspace, float* logits,
                float* x_out) {
  if (!ctx().stream) {
    set_error("plh_forward: plh_init has not been called");
    return -1;
  }
  if (!model_ok(m)) return -1;
  if (token < 0 || token >= m->vocab_size || pos < 0 || pos >= m->max_seq_len || !workspace ||
      !logits) {
    set_error("plh_forward: token %d / pos %d out of range or null buffer", token, pos);
    return -1;
  }
  return forward_token(m, token, pos, workspace, logits, x_out);
}

int plh_forward_prefill(const plh_model* m, const int* tokens, int n_tokens, int start_pos,
                        void* workspace, float* logits, float* x_out) {
  if (!ctx().stream) {
    set_error("plh_forward_prefill: plh_init has not been called");
    return -1;
  }
  if (!model_ok(m)) return -1;
  if (!tokens || n_tokens < 1 || start_pos < 0 ||
      (long)start_pos + n_tokens > (long)m->max_seq_len || !workspace || !logits) {
    set_error("plh_forward_prefill: %d tokens at %d do not fit %d positions (or null buffer)",
              n_tokens, start_pos, m->max_seq_len);
    return -1;
  }
  for (int bi = 0; bi < n_tokens; ++bi)
    if (tokens[bi] < 0 || tokens[bi] >= m->vocab_size) {
      set_error("plh_forward_prefill: token %d out of range", tokens[bi]);
      return -1;
    }
  const int chunk = min(n_tokens, kPrefillChunk);
  const ChunkActs sized = carve_chunk(m, chunk, nullptr);
  if (ensure_prefill_ws(sized.bytes)) return -1;
  const ChunkActs a = carve_chunk(m, chunk, ctx().pf_ws);
  int T = 0;
  for (int t0 = 0; t0 < n_tokens; t0 += chunk) {
    T = min(chunk, n_tokens - t0);
    if (prefill_chunk(m, tokens + t0, T, start_pos + t0, a)) return -1;
  }
  // model.c:1138-1143: final rmsnorm and logits of the last token
  const int E = m->n_embd;
  const float* xl = a.x + (size_t)(T - 1) * E;
  GemvCall g{};
  g.qtype = m->output.qtype, g.n = E, g.d = m->vocab_size, g.w = m->output.w, g.x = xl;
  g.out = logits, g.norm_w = m->output_norm, g.norm_eps = m->rms_norm_eps;
  if (E > kGemvNormMax) {  // too long for the prologue: normalise first
    if (launch_rmsnorm(xl, m->output_norm, a.xn, E, m->rms_norm_eps)) return -1;
    g.x = a.xn, g.norm_w = nullptr;
  }
  g.xn_out = g.norm_w ? x_out : nullptr;
  if (gemv_launch(g)) return -1;
  if (x_out && !g.norm_w && plh_memcpy_dtod(x_out, a.xn, (size_t)E * sizeof(float))) return -1;
  (void)workspace;
  return 0;
}

}  // extern "C"
