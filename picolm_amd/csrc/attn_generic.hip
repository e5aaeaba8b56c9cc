// attn_generic.hip -- decode and prefill attention for head dims without a
// tuned kernel (every even head_dim up to 256 but 64 and 128).
//
// Replaces the same reference code as the tuned kernels: model.c:807-892
// (decode: QK-norm, RoPE, fp16 append at row pos, online-softmax GQA
// attention over rows 0..pos) and model.c:1019-1089 (prefill: the same per
// prompt token, causal).  The reference accepts any even head_dim up to 256
// (model.c:408 sets head_dim = n_embd / n_heads; its accumulator is
// acc[256], model.c:856); the tuned kernels are built around 32-wide d blocks
// and one rope pair per lane, so other head dims run here.
//
// Two launches, both plain VALU code (these shapes are rare and small):
//   generic_append_kernel  one workgroup per (layer, token, kv head): QK-norm
//                          of k (rmsnorm in the reference's AVX2 order),
//                          RoPE with the reference's four-product rotation,
//                          the reference's fp16 rounding; cache rows are
//                          bit-identical to the reference's, and optionally
//                          mirrored into caller row buffers.
//   generic_attn_kernel    one workgroup per (layer, token, q head): q's
//                          QK-norm and RoPE into LDS, then the positions in
//                          chunks of 256 (one per thread): scores
//                          dot(q, k_t) / sqrt(head_dim), the chunk maximum,
//                          exp weights and the rescaled sums of the online
//                          softmax, v accumulated by one thread per d
//                          (scores and v sums each in four partial sums).
// The softmax is taken per chunk rather than per position, so outputs agree
// with the reference's within the attention tolerance, not bit for bit.
#include <algorithm>

#include "picolm_hip.h"
#include "attn_common.h"
#include "plh_internal.h"

namespace plh {
namespace {

constexpr int kGThreads = 256;  // = the largest head_dim: one thread per d
constexpr int kGChunk = kGThreads;
constexpr int kGMaxD = 256;
constexpr int kGSq = 8 * ((kGMaxD / 8 + 3) / 4 * 4 + 4);  // rms_sq_pitch(256) rows of 8

struct GenericArgs {
  const float* q;  // [n_launch_layers][n_tokens][n_heads*D]
  const float* k;  // [n_launch_layers][n_tokens][kv_dim]
  const float* v;
  uint16_t* kc;    // [n_layers][S][kv_dim] fp16 bits
  uint16_t* vc;
  const float* cos_t;  // [S][D/2]
  const float* sin_t;
  float* out;      // [n_launch_layers][n_tokens][out_stride]
  const float* qn;  // QK-norm weights [n_launch_layers][D], or null
  const float* kn;
  float norm_eps;
  uint16_t* k_rows;  // appended rows also here [n_launch_layers][n_tokens][kv_dim], or null
  uint16_t* v_rows;
  int layer0, n_launch_layers, n_heads, n_kv_heads, D, max_seq_len, rope_type;
  int start_pos, n_tokens, out_stride;
};

// Rope pair i of a head: (2i, 2i+1) for LLAMA, (i, i + D/2) for QWEN
// (tensor.c:583-601).
__device__ __forceinline__ void pair_of(int rope_type, int D, int i, int& i0, int& i1) {
  i0 = rope_type == PLH_ROPE_QWEN ? i : 2 * i;
  i1 = rope_type == PLH_ROPE_QWEN ? i + D / 2 : 2 * i + 1;
}

// x (global, D floats) into xs (LDS): rmsnorm(x, w) with the reference's
// rounding when w is given ((x * scale) * w, tensor.c:425-492), else a copy.
// Every thread must call it.
__device__ __forceinline__ void load_normed(const float* x, const float* w, int D, float eps,
                                            float* xs, float* sq, float* red) {
  float scale = 1.0f;
  if (w) scale = rms_scale_block<kGThreads>(x, D, eps, sq, red);
  for (int i = threadIdx.x; i < D; i += kGThreads) xs[i] = w ? (x[i] * scale) * w[i] : x[i];
  __syncthreads();
}

// Maximum (MAX) or sum of v over the workgroup; every thread gets it.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* wred) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o);
    v = MAX ? fmaxf(v, w) : v + w;
  }
  __syncthreads();  // the previous reduction's readers are done with wred
  if ((threadIdx.x & 63) == 0) wred[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = wred[0];
#pragma unroll
  for (int i = 1; i < kGThreads / 64; ++i) r = MAX ? fmaxf(r, wred[i]) : r + wred[i];
  return r;
}

// dot(q, k row) over D elements (q in LDS, the row fp16 bits in HBM): 16-byte
// loads when D is a multiple of 8 (every row offset then is too), 4-byte ones
// otherwise (D is even); four partial sums.
__device__ __forceinline__ float row_dot(const float* qs, const uint16_t* kr, int D) {
  float d4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (D % 8 == 0) {
    const uint4* kp = (const uint4*)kr;
    const int nw = D / 8;
    for (int j = 0; j < nw; j += 4) {  // four 16-byte loads issued together
      uint4 w[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) w[b] = j + b < nw ? kp[j + b] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t ws[4] = {w[b].x, w[b].y, w[b].z, w[b].w};
        const float* qq = qs + 8 * (j + b);
        if (j + b < nw) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            d4[u] = d4[u] + qq[2 * u] * f16_bits_to_f32((uint16_t)(ws[u] & 0xFFFFu));
            d4[u] = d4[u] + qq[2 * u + 1] * f16_bits_to_f32((uint16_t)(ws[u] >> 16));
          }
        }
      }
    }
  } else {
    const uint32_t* kp = (const uint32_t*)kr;
    for (int j = 0; j < D / 2; ++j) {
      const uint32_t w = kp[j];
      float& d = d4[j & 3];
      d = d + qs[2 * j] * f16_bits_to_f32((uint16_t)(w & 0xFFFFu));
      d = d + qs[2 * j + 1] * f16_bits_to_f32((uint16_t)(w >> 16));
    }
  }
  return (d4[0] + d4[1]) + (d4[2] + d4[3]);
}

__global__ __launch_bounds__(kGThreads) void generic_append_kernel(GenericArgs a) {
  __shared__ __align__(16) float sq[kGSq];
  __shared__ float red[8];
  __shared__ float kr[kGMaxD];
  const int D = a.D, kv_dim = a.n_kv_heads * D;
  const int kvh = blockIdx.x % a.n_kv_heads;
  const int t = (blockIdx.x / a.n_kv_heads) % a.n_tokens;
  const int li = blockIdx.x / (a.n_kv_heads * a.n_tokens);
  const int pos = a.start_pos + t;
  const size_t src = ((size_t)li * a.n_tokens + t) * kv_dim + (size_t)kvh * D;
  load_normed(a.k + src, a.kn ? a.kn + (size_t)li * D : nullptr, D, a.norm_eps, kr, sq, red);
  const float* cr = a.cos_t + (size_t)pos * (D / 2);
  const float* sr = a.sin_t + (size_t)pos * (D / 2);
  const size_t dst =
      ((size_t)(a.layer0 + li) * a.max_seq_len + pos) * kv_dim + (size_t)kvh * D;
  for (int i = threadIdx.x; i < D / 2; i += kGThreads) {
    int i0, i1;
    pair_of(a.rope_type, D, i, i0, i1);
    float x0 = kr[i0], x1 = kr[i1];
    rope_rotate(x0, x1, cr[i], sr[i]);
    const uint16_t b0 = f16_bits_rha(x0), b1 = f16_bits_rha(x1);
    a.kc[dst + i0] = b0;
    a.kc[dst + i1] = b1;
    if (a.k_rows) {
      a.k_rows[src + i0] = b0;
      a.k_rows[src + i1] = b1;
    }
  }
  for (int i = threadIdx.x; i < D; i += kGThreads) {
    const uint16_t b = f16_bits_rha(a.v[src + i]);
    a.vc[dst + i] = b;
    if (a.v_rows) a.v_rows[src + i] = b;
  }
}

__global__ __launch_bounds__(kGThreads) void generic_attn_kernel(GenericArgs a) {
  __shared__ float qs[kGMaxD];
  __shared__ float ps[kGChunk];
  __shared__ __align__(16) float sq[kGSq];
  __shared__ float red[8];
  __shared__ float wred[kGThreads / 64];
  const int tid = threadIdx.x;
  const int D = a.D, kv_dim = a.n_kv_heads * D, G = a.n_heads / a.n_kv_heads;
  const int h = blockIdx.x % a.n_heads;
  const int t = (blockIdx.x / a.n_heads) % a.n_tokens;
  const int li = blockIdx.x / (a.n_heads * a.n_tokens);
  const int pos = a.start_pos + t, kvh = h / G;
  const size_t row = (size_t)li * a.n_tokens + t;
  load_normed(a.q + row * a.n_heads * D + (size_t)h * D, a.qn ? a.qn + (size_t)li * D : nullptr,
              D, a.norm_eps, qs, sq, red);
  const float* cr = a.cos_t + (size_t)pos * (D / 2);
  const float* sr = a.sin_t + (size_t)pos * (D / 2);
  for (int i = tid; i < D / 2; i += kGThreads) {
    int i0, i1;
    pair_of(a.rope_type, D, i, i0, i1);
    float x0 = qs[i0], x1 = qs[i1];
    rope_rotate(x0, x1, cr[i], sr[i]);
    qs[i0] = x0;
    qs[i1] = x1;
  }
  __syncthreads();
  const size_t layer_off = (size_t)(a.layer0 + li) * a.max_seq_len * kv_dim + (size_t)kvh * D;
  const uint16_t* kl = a.kc + layer_off;
  const uint16_t* vl = a.vc + layer_off;
  const float root = sqrtf((float)D);
  float m = kNegBig, l = 0.0f, acc = 0.0f;  // acc: element d = tid of the output
  for (int c0 = 0; c0 <= pos; c0 += kGChunk) {
    const int p = c0 + tid;
    float s = kNegBig;
    if (p <= pos) s = row_dot(qs, kl + (size_t)p * kv_dim, D) / root;
    const float mn = fmaxf(m, block_reduce<true>(s, wred));
    const float e = p <= pos ? expf(s - mn) : 0.0f;
    ps[tid] = e;
    const float esum = block_reduce<false>(e, wred);  // its barriers publish ps
    const float corr = expf(m - mn);
    l = l * corr + esum;
    if (tid < D) {
      const int np = min(kGChunk, pos + 1 - c0);
      const uint16_t* vp = vl + (size_t)c0 * kv_dim + tid;
      // eight v loads in flight, four independent partial sums
      float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      int j = 0;
      for (; j + 8 <= np; j += 8) {
        uint16_t vb[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) vb[u] = vp[(size_t)(j + u) * kv_dim];
#pragma unroll
        for (int u = 0; u < 8; ++u) s4[u & 3] = s4[u & 3] + ps[j + u] * f16_bits_to_f32(vb[u]);
      }
      for (; j < np; ++j) s4[0] = s4[0] + ps[j] * f16_bits_to_f32(vp[(size_t)j * kv_dim]);
      acc = acc * corr + ((s4[0] + s4[1]) + (s4[2] + s4[3]));
    }
    m = mn;
    __syncthreads();  // ps is rewritten by the next chunk
  }
  if (tid < D) a.out[row * a.out_stride + (size_t)h * D + tid] = acc / l;
}

}  // namespace

int attn_generic(int n_heads, int n_kv_heads, int head_dim, int max_seq_len, int rope_type,
                 int layer0, int n_launch_layers, int start_pos, int n_tokens, const float* q,
                 const float* k, const float* v, uint16_t* key_cache, uint16_t* val_cache,
                 const float* rope_cos, const float* rope_sin, float* out, int out_stride,
                 const float* q_norm, const float* k_norm, float norm_eps, uint16_t* k_rows,
                 uint16_t* v_rows) {
  if (head_dim < 2 || head_dim > kGMaxD || head_dim % 2) {
    set_error("attention: head_dim %d must be even and at most %d", head_dim, kGMaxD);
    return -1;
  }
  if (n_tokens == 0) return 0;
  GenericArgs a;
  a.q = q, a.k = k, a.v = v, a.kc = key_cache, a.vc = val_cache;
  a.cos_t = rope_cos, a.sin_t = rope_sin, a.out = out;
  a.qn = q_norm, a.kn = k_norm, a.norm_eps = norm_eps;
  a.k_rows = k_rows, a.v_rows = v_rows;
  a.layer0 = layer0, a.n_launch_layers = n_launch_layers, a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads, a.D = head_dim, a.max_seq_len = max_seq_len;
  a.rope_type = rope_type, a.start_pos = start_pos, a.n_tokens = n_tokens;
  a.out_stride = out_stride;
  // A launch holds at most 2^32 - 1 threads: layers go in as many launches
  // as that takes (each layer is independent); one layer must fit.
  const long per_layer = (long)n_tokens * n_heads;
  const long max_wg = 0xFFFFFFFFL / kGThreads;
  if (per_layer > max_wg) {
    set_error("attention: %d tokens x %d heads exceed one launch's %ld workgroups", n_tokens,
              n_heads, max_wg);
    return -1;
  }
  const int step = (int)std::min<long>(n_launch_layers, max_wg / per_layer);
  const size_t q_dim = (size_t)n_heads * head_dim, kv_dim = (size_t)n_kv_heads * head_dim;
  hipStream_t st = ctx().stream;
  for (int l = 0; l < n_launch_layers; l += step) {
    GenericArgs b = a;
    const size_t rows_before = (size_t)l * n_tokens;
    b.layer0 = layer0 + l;
    b.n_launch_layers = std::min(step, n_launch_layers - l);
    b.q = q + rows_before * q_dim;
    b.k = k + rows_before * kv_dim;
    b.v = v + rows_before * kv_dim;
    b.out = out + rows_before * out_stride;
    if (q_norm) b.qn = q_norm + (size_t)l * head_dim;
    if (k_norm) b.kn = k_norm + (size_t)l * head_dim;
    if (k_rows) b.k_rows = k_rows + rows_before * kv_dim;
    if (v_rows) b.v_rows = v_rows + rows_before * kv_dim;
    const long nl = b.n_launch_layers;
    hipLaunchKernelGGL(generic_append_kernel, dim3((unsigned)(nl * n_tokens * n_kv_heads)),
                       dim3(kGThreads), 0, st, b);
    if (check_hip(hipGetLastError(), "generic_append_kernel")) return -1;
    hipLaunchKernelGGL(generic_attn_kernel, dim3((unsigned)(nl * per_layer)), dim3(kGThreads), 0,
                       st, b);
    if (check_hip(hipGetLastError(), "generic_attn_kernel")) return -1;
  }
  return 0;
}

}  // namespace plh
