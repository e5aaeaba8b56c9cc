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

namespace {

constexpr int kTypeF32 = 0, kTypeF16 = 1, kTypeQ4_0 = 2, kTypeQ8_0 = 8, kTypeQ4K = 12,
              kTypeQ6K = 14;
constexpr int kNormThreads = 256;
constexpr int kMaxNormSize = 12288;  // the squares of a row must fit 48 KiB of LDS

// ---- rmsnorm (tensor.c:425-492, x86-64 AVX2 path) --------------------------
// The reference keeps eight lane sums acc[j] += x[8i+j]^2 (product, then
// sum) over i in order, folds them as ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)),
// adds the tail x[i]^2 for i >= 8*(n/8) one by one, takes
// 1/sqrtf(ss/n + eps) and writes (x*scale)*w.  Here the workgroup squares x
// into LDS transposed (chain j's squares contiguous), eight lanes run the
// eight chains, lane 0 folds, and every thread writes its outputs.  Device
// division and square root are correctly rounded, so the scale is the
// reference's bit for bit.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* x, const float* w,
                                                               float* out, int n, float eps) {
  extern __shared__ __align__(16) float sq[];
  __shared__ float chain[8];
  __shared__ float scale_s;
  const int tid = threadIdx.x;
  const int n8 = n / 8;
  const int pitch = (n8 + 3) / 4 * 4 + 4;
  for (int idx = tid; idx < 8 * n8; idx += kNormThreads) {
    const float v = x[idx];
    sq[(idx & 7) * pitch + (idx >> 3)] = v * v;
  }
  __syncthreads();
  if (tid < 8) {
    const float* s = sq + tid * pitch;
    float acc = 0.0f;
    int i = 0;
    for (; i + 4 <= n8; i += 4) {
      const float4 v = *(const float4*)(s + i);
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
    }
    for (; i < n8; ++i) acc = acc + s[i];
    chain[tid] = acc;
  }
  __syncthreads();
  if (tid == 0) {
    const float l0 = chain[0] + chain[4], l1 = chain[1] + chain[5];
    const float l2 = chain[2] + chain[6], l3 = chain[3] + chain[7];
    float ss = (l0 + l2) + (l1 + l3);
    for (int i = 8 * n8; i < n; ++i) ss = ss + x[i] * x[i];
    scale_s = 1.0f / sqrtf(ss / (float)n + eps);
  }
  __syncthreads();
  const float scale = scale_s;
  for (int i = tid; i < n; i += kNormThreads) {
    const float t = x[i] * scale;
    out[i] = t * w[i];
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

__global__ __launch_bounds__(256) void dequant_row_kernel(int qtype, const uint8_t* row,
                                                          float* out, int n) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
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
  out[e] = y;
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

size_t norm_lds_bytes(int n) { return sizeof(float) * 8 * (size_t)((n / 8 + 3) / 4 * 4 + 4); }

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
  const size_t wide = q_dim > (size_t)m->n_embd ? q_dim : (size_t)m->n_embd;
  const size_t sizes[7] = {(size_t)m->n_embd, wide, q_dim, kv_dim, kv_dim, q_dim, (size_t)m->n_ffn};
  float** dst[7];
  Acts a{};
  dst[0] = &a.x, dst[1] = &a.xb, dst[2] = &a.q, dst[3] = &a.k, dst[4] = &a.v, dst[5] = &a.att,
  dst[6] = &a.hb;
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
      m->n_heads % m->n_kv_heads || (m->head_dim != 64 && m->head_dim != 128) ||
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

int plh_forward(const plh_model* m, int token, int pos, void* workspace, float* logits,
                float* x_out) {
  Context& c = ctx();
  if (!c.stream) {
    set_error("plh_forward: plh_init has not been called");
    return -1;
  }
  if (!model_ok(m)) return -1;
  if (token < 0 || token >= m->vocab_size || pos < 0 || pos >= m->max_seq_len || !workspace ||
      !logits) {
    set_error("plh_forward: token %d / pos %d out of range or null buffer", token, pos);
    return -1;
  }
  const int E = m->n_embd, F = m->n_ffn;
  const int Q = m->n_heads * m->head_dim, KV = m->n_kv_heads * m->head_dim;
  const float eps = m->rms_norm_eps;
  const Acts a = carve(m, workspace);
  const size_t rb = embd_row_bytes(m->embd_type, E);
  if (plh_dequantize_row(m->embd_type, (const uint8_t*)m->token_embd + (size_t)token * rb, a.x,
                         E))
    return -1;
  for (int l = 0; l < m->n_layers; ++l) {
    const plh_layer& L = m->layers[l];
    // attention block (model.c:777-897)
    if (launch_rmsnorm(a.x, L.attn_norm, a.xb, E, eps)) return -1;
    if (plh_gemv_ex(L.q.qtype, E, Q, L.q.w, a.xb, a.q, L.q_bias, L.q_bias == nullptr, nullptr,
                    nullptr) ||
        plh_gemv_ex(L.k.qtype, E, KV, L.k.w, a.xb, a.k, L.k_bias, 0, nullptr, nullptr) ||
        plh_gemv_ex(L.v.qtype, E, KV, L.v.w, a.xb, a.v, L.v_bias, 0, nullptr, nullptr))
      return -1;
    const int rc = L.q_norm ? plh_attn_decode_qknorm(m->n_layers, m->n_heads, m->n_kv_heads,
                                                     m->head_dim, m->max_seq_len, m->rope_type, l,
                                                     1, pos, a.q, a.k, a.v, m->key_cache,
                                                     m->val_cache, m->rope_cos, m->rope_sin,
                                                     a.att, L.q_norm, L.k_norm, eps)
                            : plh_attn_decode(m->n_layers, m->n_heads, m->n_kv_heads,
                                              m->head_dim, m->max_seq_len, m->rope_type, l, 1,
                                              pos, a.q, a.k, a.v, m->key_cache, m->val_cache,
                                              m->rope_cos, m->rope_sin, a.att);
    if (rc) return -1;
    // x = x + (Wo att + o_bias)
    if (plh_gemv_ex(L.o.qtype, Q, E, L.o.w, a.att, a.x, L.o_bias, L.o_bias == nullptr, nullptr,
                    a.x))
      return -1;
    // SwiGLU block (model.c:899-922)
    if (launch_rmsnorm(a.x, L.ffn_norm, a.xb, E, eps)) return -1;
    if (plh_gemv_ex(L.gate.qtype, E, F, L.gate.w, a.xb, a.hb, nullptr, 0, nullptr, nullptr) ||
        plh_gemv_ex(L.up.qtype, E, F, L.up.w, a.xb, a.hb, nullptr, 0, a.hb, nullptr) ||
        plh_gemv_ex(L.down.qtype, F, E, L.down.w, a.hb, a.x, nullptr, 0, nullptr, a.x))
      return -1;
  }
  // final norm and logits (model.c:918-922)
  if (launch_rmsnorm(a.x, m->output_norm, a.xb, E, eps)) return -1;
  if (plh_gemv_ex(m->output.qtype, E, m->vocab_size, m->output.w, a.xb, logits, nullptr, 0,
                  nullptr, nullptr))
    return -1;
  if (x_out && plh_memcpy_dtod(x_out, a.xb, (size_t)E * sizeof(float))) return -1;
  return 0;
}

}  // extern "C"
