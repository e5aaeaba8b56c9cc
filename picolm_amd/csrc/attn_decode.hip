// attn_decode.hip -- single-token decode attention for gfx950.
//
// Replaces model.c:819-892: RoPE of q and k with table row `pos`, append of
// f16(k_rot), f16(v) at cache row `pos`, and the online-softmax GQA attention
// over rows 0..pos.  One launch may cover several layers (each layer is an
// independent problem; the bench's all-layers step uses this).
//
// Work decomposition.  A "group" is (layer, kv head, block of <=16 q heads of
// that kv head's GQA group); the group's positions are cut into `n_split`
// splits of `split_len` rows; a workgroup (4 wavefronts) owns one (group,
// split) unit and its waves take 32-row tiles of the split in turn, keeping
// the loads of the next tile in flight while one tile is computed.
// Splits are short (512-1024 rows) and numerous (several workgroups per CU):
// on MI355X one CU streams only ~35 GB/s, so reaching HBM bandwidth needs
// nearly every CU streaming, and small register-light workgroups keep several
// per CU in flight to cover each one's q-load latency.  Deeper per-wave
// prefetch measured slower.  Every K/V
// byte of the group is read from HBM exactly once, whatever the GQA factor,
// because all q heads of the group ride in the same MFMA.
//
// Per 32-row tile, per wave:
//   S^T[t][h] = K[t][:] . q[h][:]   two v_mfma_f32_16x16x32_f16 row blocks,
//                                   q split into fp16 hi+lo (two MFMAs each)
//                                   so the product keeps ~fp32 precision;
//   online softmax in the log2 domain: maximum over raw scores, scale folded
//                                   into the exp2 argument (rounded product
//                                   minus the running maximum: monotone, so
//                                   weights stay bounded at any score
//                                   magnitude), rescale of O only when the
//                                   maximum grows by more than 2^8;
//   O^T[d][h] += V^T[d][t] P^T[t][h] with P split hi+lo; V goes row-major
//                                   through a per-wave LDS tile and comes back
//                                   transposed by ds_read_b64_tr_b16;
//   the softmax denominators ride in the same MFMA pipe (ones . P^T).
// The S^T accumulator layout (lane = 16*g + h holds rows 4g..4g+3 of each
// 16-row block) is used directly as the B operand of the PV product: the
// K slots (g, j) of that product map to tile rows 4g+j (j<4) and 16+4g+j-4
// (j>=4); the two transposing reads of a 16-column block fetch exactly those
// rows.
//
// Row `pos` itself is never read back from the cache: the workgroup owning
// the last split computes k_rot/v for that row, writes the fp16 row, and
// folds it into its result as one extra softmax partial.  No workgroup reads
// memory another one writes, except the split partials below.
//
// Split combine: each workgroup merges its 4 waves (and the new row) through
// LDS.  With one split it writes the normalised output.  Otherwise it stores
// (max, sum, acc[D]) per head to the workspace and a second, small kernel on
// the same stream merges the splits of each group.  No workgroup waits on
// another: on gfx950 an agent-scope release fence writes back the XCD's whole
// L2, and a last-arriving-workgroup merge (one such fence per workgroup)
// measured several times slower than the second launch.
#include <math.h>

#include "attn_common.h"
#include "picolm_hip.h"
#include "plh_internal.h"

using namespace plh;

// ---- static scratch of the allocation-free entry point ---------------------
// plh_attn_decode_noalloc keeps its split partials in this file-scope device
// array instead of the library workspace: each GPU holds its own copy until
// the process ends, and every call on a GPU shares it (concurrent calls on one
// GPU would race; the library's single stream serialises its own calls).  No
// part of it needs clearing: every partial a launch reads was written by the
// same launch.  In host code `scratch` is a host-side stand-in, not a device
// address: decode_scratch_setup (called by plh_init with the device current)
// looks the device address up once per device, and launches use that.
static constexpr size_t kScratchBytes = 16u << 20;
// its first kScratchCounterBytes hold the stream-K kernel's arrival counters,
// the rest the split partials
static constexpr size_t kScratchCounterBytes = (size_t)kDecodeCounters * sizeof(unsigned);
static constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static void* g_scratch_ptr[kMaxDevices];  // its device address, per device

#include "attn_decode_dev.h"

namespace {

template <int D, bool QKN>
__global__ __launch_bounds__(64 * DecodeShape<D>::W) void attn_decode_kernel(DecodeArgs a) {
  attn_decode_body<D, QKN, false>(a, PfLaunch{});
}
template <int D, bool QKN>
__global__ __launch_bounds__(64 * DecodeShape<D>::W) void attn_decode_pf_kernel(DecodeArgs a,
                                                                               PfLaunch pl) {
  attn_decode_body<D, QKN, true>(a, pl);
}

// Merges the n_split partials of one group: out = sum_s O_s 2^(m_s-M) /
// sum_s l_s 2^(m_s-M) with M the largest m_s.  CH partials are loaded
// together (8 when there are at most 8 splits, else kCombineChunk).
template <int D, int CH>
__global__ __launch_bounds__(kCombineThreads) void attn_decode_combine_kernel(DecodeArgs a) {
  // group g runs on the XCD whose L2 holds its partials: the main kernel put
  // group g's splits on XCD g / (per_xcd / n_split), and consecutive
  // workgroup ids go to consecutive XCDs
  const int gpx = a.per_xcd / a.n_split;
  const int group = (int)(blockIdx.x & 7) * gpx + (int)(blockIdx.x >> 3);
  if (group * a.n_split >= a.n_units) return;
  const int gh = (int)fdiv(group, a.fd_hblk);  // group / n_hblk
  const int hblk = group - gh * a.n_hblk;
  const int li = (int)fdiv(gh, a.fd_kvh);
  const int kvh = gh - li * a.n_kv_heads;
  const int G = a.G;
  const int h0 = hblk * 16;
  const int nh = min(16, G - h0);
  float* out_base = a.out + (size_t)li * a.n_heads * D + (size_t)(kvh * G + h0) * D;
  const int u0 = group * a.n_split;
  // blockIdx.y slices the group's (head, d) elements: one element per thread,
  // so each thread's loads make a single memory round trip
  for (int idx = blockIdx.y * kCombineThreads + threadIdx.x; idx < nh * D;
       idx += kCombineThreads * gridDim.y) {
    const int h = idx / D, d = idx - (idx / D) * D;
    // the loads of a chunk of splits are issued together, then merged
    float M = kNegBig, L = 0.f, O = 0.f;
    for (int s0 = 0; s0 < a.n_split; s0 += CH) {
      float mi[CH], li[CH], oi[CH];
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const size_t u = (size_t)(u0 + min(s0 + j, a.n_split - 1)) * a.nhm + h;
        mi[j] = a.part_m[u];
        li[j] = a.part_l[u];
        oi[j] = a.part_o[u * D + d];
      }
      float Mc = M;
#pragma unroll
      for (int j = 0; j < CH; ++j)
        if (s0 + j < a.n_split) Mc = fmaxf(Mc, mi[j]);
      const float r = fast_exp2(M - Mc);
      L *= r;
      O *= r;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        if (s0 + j < a.n_split) {
          const float w = fast_exp2(mi[j] - Mc);
          L = __builtin_fmaf(li[j], w, L);
          O = __builtin_fmaf(oi[j], w, O);
        }
      }
      M = Mc;
    }
    out_base[(size_t)h * D + d] = O * (1.0f / L);
  }
}

template <int D, bool QKN, int kSkPF>
__global__ __launch_bounds__(256) void attn_decode_sk_kernel(DecodeArgs a) {
  attn_decode_sk_body<D, QKN, kSkPF, false>(a, PfLaunch{});
}
// with prefetch workgroups: the default two tiles in flight only
template <int D, bool QKN>
__global__ __launch_bounds__(256) void attn_decode_sk_pf_kernel(DecodeArgs a, PfLaunch pl) {
  attn_decode_sk_body<D, QKN, 2, true>(a, pl);
}

// Split plan defaults, from sweeps on MI355X (TinyLlama pos 256 and 2047,
// Llama-3.2 pos 8191, Llama-2 pos 4095, one-layer launches): about four
// workgroups per CU; contexts up to 512 positions are not split.
constexpr int kDefaultMinSplit = 512;
int g_target_units = 0;   // 0: four workgroups per CU
int g_min_split = kDefaultMinSplit;
int g_decode_kernel = 0;  // plh_set_tuning key 7: 0 by shape, 1 split + combine, 2 stream-K
int g_sk_workgroups = 0;  // key 8: stream-K workgroups (0: the launch's own choice)
int g_sk_pf = 0;          // key 9: stream-K tiles in flight per wave (0: by head_dim)
int g_sk_xcd_local = 0;   // key 11: XCD-local stream-K merges (0 by shape, 1 always, -1 never)
int g_split_merge = 0;    // key 14: the split kernel merges in the launch (0) or a combine launch (-1)

// Each workgroup's XCD (the hardware XCC_ID register) by workgroup id.
constexpr int kXcdProbeGroups = 2048;
__global__ __launch_bounds__(64) void xcd_probe_kernel(unsigned* out) {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  if (threadIdx.x == 0) out[blockIdx.x] = x;
}

}  // namespace

namespace plh {
// key 15: the forward's attention launches prefetch the o-projection's, the
// gate/up pair's and the down projection's weights (0), the first two only
// (1), or none (-1)
int g_fwd_prefetch = 0;
int g_fwd_fuse = 0;  // key 17
int g_xcd_ok[kMaxDevices] = {};

int decode_scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices) {
    set_error("plh_init: device %d beyond the %d the static scratch table covers", device,
              kMaxDevices);
    return -1;
  }
  if (g_scratch_ptr[device]) return 0;
  void* p = nullptr;
  if (check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
    return -1;
  // the stream-K merge counters at the start of the array start at zero
  // (every launch leaves them zero again)
  Context& c = ctx();
  if (check_hip(hipMemsetAsync(p, 0, kScratchCounterBytes, c.stream), "hipMemsetAsync(scratch)") ||
      check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize"))
    return -1;
  // The stream-K kernel's XCD-local merges need every workgroup id
  // congruent mod 8 to run on one XCD (the dispatcher deals workgroups to
  // the XCDs in turn); the ids' XCDs are read back once per device, through
  // the scratch's partial region, and the merges stay device-wide otherwise.
  unsigned* probe = (unsigned*)((char*)p + kScratchCounterBytes);
  unsigned xcc[kXcdProbeGroups];
  hipLaunchKernelGGL(xcd_probe_kernel, dim3(kXcdProbeGroups), dim3(64), 0, c.stream, probe);
  if (check_hip(hipGetLastError(), "xcd_probe_kernel") ||
      check_hip(hipMemcpyAsync(xcc, probe, sizeof(xcc), hipMemcpyDeviceToHost, c.stream),
                "hipMemcpyAsync(xcd probe)") ||
      check_hip(hipStreamSynchronize(c.stream), "hipStreamSynchronize"))
    return -1;
  bool same = true;
  for (int b = 8; b < kXcdProbeGroups; ++b) same = same && xcc[b] == xcc[b & 7];
  g_xcd_ok[device] = same ? 1 : -1;
  g_scratch_ptr[device] = p;
  return 0;
}
}  // namespace plh

extern "C" int plh_set_tuning(int key, int value) {
  if (key == 1) {
    g_target_units = value < 0 ? 0 : value;
    return 0;
  }
  if (key == 2) {
    if (value == 0) {
      g_min_split = kDefaultMinSplit;
      return 0;
    }
    if (value < 128 || value % 128) {
      set_error("plh_set_tuning: minimum split must be a positive multiple of 128");
      return -1;
    }
    g_min_split = value;
    return 0;
  }
  if (key == 3) {
    if (value != 0 && value != 1 && value != 2 && value != 4 && value != 8) {
      set_error("plh_set_tuning: GEMV rows per thread must be 0, 1, 2, 4 or 8");
      return -1;
    }
    g_gemv_rows_per_thread = value;
    return 0;
  }
  if (key == 4) {
    if (value != 0 && value != 1) {
      set_error("plh_set_tuning: forward rmsnorm placement must be 0 or 1");
      return -1;
    }
    g_fwd_norm_separate = value;
    return 0;
  }
  if (key == 5) {
    if (value != 0 && value != -1 && value != 2 && value != 4 && value != 8 && value != 16) {
      set_error("plh_set_tuning: prefill chunking must be 0, -1, 2, 4, 8 or 16");
      return -1;
    }
    g_prefill_split = value;
    return 0;
  }
  if (key == 6) {
    if (value != 0 && value != -1 && value != 2 && value != 3) {
      set_error("plh_set_tuning: prefill K-split must be 0, -1, 2 or 3");
      return -1;
    }
    g_prefill_ksplit = value;
    return 0;
  }
  if (key == 7) {
    if (value != 0 && value != 1 && value != 2) {
      set_error("plh_set_tuning: decode kernel must be 0 (by shape), 1 (split + combine) or 2 "
                "(stream-K)");
      return -1;
    }
    g_decode_kernel = value;
    return 0;
  }
  if (key == 8) {
    if (value < 0) {
      set_error("plh_set_tuning: stream-K workgroups must be >= 0");
      return -1;
    }
    g_sk_workgroups = value;
    return 0;
  }
  if (key == 10) {
    if (value != 0 && value != 1) {
      set_error("plh_set_tuning: GEMV order must be 0 (fast) or 1 (exact)");
      return -1;
    }
    g_gemv_exact = value;
    return 0;
  }
  if (key == 14) {
    if (value != 0 && value != -1) {
      set_error("plh_set_tuning: split merge must be 0 (in the launch) or -1 (combine launch)");
      return -1;
    }
    g_split_merge = value;
    return 0;
  }
  if (key == 15) {
    if (value < -1 || value > 1) {
      set_error("plh_set_tuning: forward weight prefetch must be 0, 1 or -1 (off)");
      return -1;
    }
    g_fwd_prefetch = value;
    return 0;
  }
  if (key == 17) {
    if (value < -1 || value > kPfMaxPerXcd || (value > 0 && value < 8)) {
      set_error("plh_set_tuning: forward q/k/v + attention fusion must be -1, 0 or 8..31");
      return -1;
    }
    g_fwd_fuse = value;
    return 0;
  }
  if (key == 11) {
    if (value < -1 || value > 1) {
      set_error("plh_set_tuning: XCD-local stream-K merges must be 0 (by shape), 1 or -1");
      return -1;
    }
    g_sk_xcd_local = value;
    return 0;
  }
  if (key == 9) {
    if (value != 0 && value != 2 && value != 3 && value != 4) {
      set_error("plh_set_tuning: stream-K prefetch depth must be 0, 2, 3 or 4");
      return -1;
    }
    g_sk_pf = value;
    return 0;
  }
  set_error("plh_set_tuning: unknown key %d", key);
  return -1;
}

// Which decode kernel a launch gets (plh_set_tuning key 7 overrides).
// Measured on MI355X with all layers in one launch and with one launch per
// layer: the stream-K kernel is faster for head_dim 128 (Llama-2 pos 4095:
// 355 against 379 us per token, per-layer 601 against 778 us) and for
// head_dim 64 ranges of at most 64 blocks per workgroup (TinyLlama pos
// 2047: 16.7-17.2 against 17.6-17.9 us); the split kernel is faster for long
// head_dim 64 streams (Llama-3.2 pos 8191, 256 blocks per workgroup: 54.9
// against 61.9 us) and for contexts it does not split (TinyLlama pos 256:
// 6.6 against 8.3 us).
// Stream-K workgroups of a launch (tuning key 8 overrides).  Head_dim 64
// launches whose groups split evenly over the XCDs take an aligned plan:
// W = k * n_groups, so each workgroup streams 1/k of one group and a
// group's k producers sit on one XCD (merged through its L2), with k the
// smallest power of two that gives about 0.6 workgroups per CU or more and
// at most 384 KB of K and V rows per workgroup (W at most 4 per CU and at
// least 8 blocks a range, else the general plan).  Measured on MI355X, all-layer TinyLlama launches (88
// groups): pos 512 / 600 / 1024 / 2047 took 8.2 / 8.7 / 10.0 / 15.6 us with
// k = 2 against 12.0 / 11.9 / 13.4 / 16.4 us for the general plan;
// Llama-3.2 (128 groups) pos 4095 / 8191 33.2 / 56.1 us with k = 4 / 8
// against 33.9 / 63.8 us (those launches run the split kernel, 31.5 / 55.2
// us).  Otherwise about one workgroup per CU, each with at least 8
// blocks (one 32-row tile per wave): head_dim 128 launches gain nothing
// from the aligned plan (Qwen3 pos 2047: 50.1-51.3 us with k = 1 and
// 52.9-59.8 us with k = 2 or 4, against 51.5 us).
//
// Launches whose groups do not split evenly over the XCDs (one TinyLlama
// layer: 4 groups) take an aligned plan too, merged device-wide: k at most 8
// ranges a group (one round of partial loads) of at least 8 blocks each,
// the fewest that give ~0.6 workgroups per CU, else the most allowed.  One
// TinyLlama layer at pos 700 / 1024 / 2047: 168 / 163 / 179 us per token
// with k = 4 / 8 / 8, against 243 / 162 / 184 us for the general plan.
//
// Otherwise the general plan's workgroup count, rounded down to a
// power-of-two number of ranges per group when it covers every group once
// (aligned), else cut over the flattened blocks.
//
// Aligned plans give every group its own k ranges (*k_out = k); the
// general plan cuts the flattened blocks (*k_out = 0).
static long sk_plan_workgroups(int head_dim, int n_groups, int nbk, int num_cus, int device,
                               int* k_out) {
  const long T = (long)n_groups * nbk;
  const long cus = num_cus > 0 ? num_cus : 256;
  *k_out = 0;
  if (g_sk_workgroups > 0) return g_sk_workgroups;
  if (head_dim == 64 && n_groups % 8 == 0 && g_sk_xcd_local >= 0 && g_xcd_ok[device] == 1) {
    const double bytes = (double)T * 16 * 64 * 2 * 2;  // K and V rows the launch reads
    for (long k = 1; k <= nbk / 8 && k * n_groups <= 4 * cus; k *= 2)
      if (k * n_groups * 10 >= 6 * cus && bytes / (double)(k * n_groups) <= 384.0 * 1024) {
        *k_out = (int)k;
        return k * n_groups;
      }
  }
  if (head_dim == 64 && (long)n_groups * 10 < 6 * cus) {
    int cap = 0;
    for (int k = 2; k <= 8 && nbk / k >= 8; k *= 2) cap = k;
    if (cap >= 2) {
      int k = 2;
      while (k < cap && (long)k * n_groups * 10 < 6 * cus) k *= 2;
      *k_out = k;
      return (long)k * n_groups;
    }
  }
  long W = T / 8;
  if (W > cus) W = cus;
  // the general plan's count, aligned: the largest power-of-two number of
  // ranges a group it allows (Qwen3 28 layers at pos 700: 23.5 -> 17.9 us)
  if (W >= n_groups) {
    int k = 1;
    while ((long)2 * k * n_groups <= W) k *= 2;
    *k_out = k;
    return (long)k * n_groups;
  }
  return W;
}

static bool use_stream_k(int head_dim, int pos, int n_groups, int num_cus) {
  if (g_decode_kernel) return g_decode_kernel == 2;
  if (pos + 1 <= g_min_split) return false;
  if (head_dim == 128) return true;
  // by the general plan's range length (the aligned plan's would send
  // Llama-3.2 pos 4095 to stream-K: 32.5 us against 31.5 us split)
  const long T = (long)n_groups * ((pos + 15) / 16);
  const long cus = num_cus > 0 ? num_cus : 256;
  long W = T / 8;
  if (W > cus) W = cus;
  return W > 0 && T / W <= 64;
}

// Plans and queues one stream-K launch (attn_decode_sk_kernel).
// The stream-K launch's plan and arguments (W workgroups).
static int sk_prepare(int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                      int rope_type, int layer0, int n_launch_layers, int pos, const float* q,
                      const float* k, const float* v, uint16_t* key_cache, uint16_t* val_cache,
                      const float* rope_cos, const float* rope_sin, float* out,
                      const float* q_norm, const float* k_norm, float norm_eps, bool noalloc,
                      uint16_t* k_rows, uint16_t* v_rows, DecodeArgs& a, long* W_out) {
  Context& c = ctx();
  const int G = n_heads / n_kv_heads;
  const int n_hblk = (G + 15) / 16;
  const int nhm = G < 16 ? G : 16;
  const int n_groups = n_launch_layers * n_kv_heads * n_hblk;
  // cached rows [0, pos) in 16-row blocks (one empty block at pos 0)
  const int nbk = pos > 0 ? (pos + 15) / 16 : 1;
  const long T = (long)n_groups * nbk;
  if (T > 0x7fffffffL) {
    set_error("plh_attn_decode: %ld cache blocks in one launch exceed the 32-bit plan", T);
    return -1;
  }
  const int cus = c.num_cus > 0 ? c.num_cus : 256;
  int k_aligned = 0;
  long W = sk_plan_workgroups(head_dim, n_groups, nbk, cus, c.device, &k_aligned);
  if (W > T) W = T;
  if (W < 1) W = 1;
  // producers per group (the partial slots it needs)
  int maxp = k_aligned;
  if (!k_aligned) {
    maxp = 1;
    const long qq = T / W, rr = T % W, big = rr * (qq + 1);
    auto owner_of = [&](long t) { return t < big ? t / (qq + 1) : rr + (t - big) / qq; };
    for (int g = 0; g < n_groups; ++g) {
      const long gb = (long)g * nbk;
      const long np = owner_of(gb + nbk - 1) - owner_of(gb) + 1;
      if (np > maxp) maxp = (int)np;
    }
  }
  const size_t part_bytes =
      maxp > 1 ? (size_t)n_groups * maxp * nhm * (head_dim + 4) * sizeof(float) : 16;
  float* part;
  unsigned* ctr;
  if (noalloc) {
    if (part_bytes > kScratchBytes - kScratchCounterBytes) {
      set_error("plh_attn_decode_noalloc: this launch needs %zu bytes of split partials, "
                "more than the %zu bytes the static scratch holds for them",
                part_bytes, kScratchBytes - kScratchCounterBytes);
      return -1;
    }
    ctr = (unsigned*)g_scratch_ptr[c.device];
    part = (float*)((char*)g_scratch_ptr[c.device] + kScratchCounterBytes);
  } else {
    if (part_bytes > 0x7fffffffu) {
      set_error("plh_attn_decode: %zu bytes of split partials exceed the 2 GiB buffer range",
                part_bytes);
      return -1;
    }
    if (ensure_workspace(part_bytes)) return -1;
    ctr = c.decode_ctr;
    part = (float*)c.ws;
  }

  a = DecodeArgs{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.kc = key_cache;
  a.vc = val_cache;
  a.cos_t = rope_cos;
  a.sin_t = rope_sin;
  a.out = out;
  a.layer0 = layer0;
  a.n_launch_layers = n_launch_layers;
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.max_seq_len = max_seq_len;
  a.pos = pos;
  a.rope_type = rope_type;
  a.n_hblk = n_hblk;
  a.nhm = nhm;
  a.qn = q_norm;
  a.kn = k_norm;
  a.norm_eps = norm_eps;
  a.score_scale = kLog2e / sqrtf((float)head_dim);
  a.k_rows = k_rows;
  a.v_rows = v_rows;
  a.sk_q = (int)(T / W);
  a.sk_r = (int)(T % W);
  a.sk_nbk = nbk;
  a.G = G;
  a.fd_hblk = make_fastdiv((uint32_t)n_hblk);
  a.fd_kvh = make_fastdiv((uint32_t)n_kv_heads);
  a.fd_nbk = make_fastdiv((uint32_t)nbk);
  // q = 0 (fewer blocks than workgroups) never divides by q: every block
  // then lies in the first r ranges
  a.fd_q = make_fastdiv((uint32_t)(a.sk_q > 0 ? a.sk_q : 1));
  a.fd_q1 = make_fastdiv((uint32_t)(a.sk_q + 1));
  // Ranges dealt to the XCDs in blocks, so that groups whose producers all
  // land on one XCD merge through its L2: needs workgroups that split evenly
  // over the eight XCDs, the local counters to fit, and plh_init's check
  // that workgroup ids congruent mod 8 share an XCD.  By shape (measured on
  // MI355X, one launch per layer and all layers in one): head_dim 64 always
  // (TinyLlama pos 1024 14.3 -> 13.3 us, pos 2047 16.5 -> 16.1 us, per layer
  // 190.6 -> 185.9 us per token; Llama-3.2 pos 8191 per layer 218 -> 162
  // us); head_dim 128 only with 16 or more workgroups per group, where the
  // merge dominates (Qwen3 pos 2047 per layer 341 -> 313 us, a 16-layer
  // 8-kv-head model at pos 8191 per layer 289 -> 268 us).  Fewer producers
  // per group at head_dim 128 lose more to the XCD-major placement of the
  // ranges than the L2 merge saves (Llama-2 pos 4095: 355 -> 361 us, per
  // layer 594 -> 640 us).
  const bool xcd_shape = g_sk_xcd_local > 0 || head_dim == 64 || W >= 16L * n_groups;
  const bool xcd_local = g_sk_xcd_local >= 0 && xcd_shape && g_xcd_ok[c.device] == 1 &&
                         W % 8 == 0 && W >= 16;
  a.sk_wx = xcd_local ? (int)(W / 8) : 0;
  a.fd_wx = make_fastdiv((uint32_t)(xcd_local ? W / 8 : 1));
  a.sk_k = k_aligned;
  a.sk_kshift = 0;
  while ((1 << a.sk_kshift) < k_aligned) ++a.sk_kshift;
  a.sk_maxp = maxp;
  a.sk_groups = n_groups;
  a.sk_part = part;
  a.sk_part_bytes = (uint32_t)part_bytes;
  a.sk_ctr = ctr;
  *W_out = W;
  return 0;
}

static int attn_decode_sk_launch(int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                                 int rope_type, int layer0, int n_launch_layers, int pos,
                                 const float* q, const float* k, const float* v,
                                 uint16_t* key_cache, uint16_t* val_cache, const float* rope_cos,
                                 const float* rope_sin, float* out, const float* q_norm,
                                 const float* k_norm, float norm_eps, bool noalloc,
                                 uint16_t* k_rows, uint16_t* v_rows) {
  Context& c = ctx();
  DecodeArgs a;
  long W;
  if (sk_prepare(n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
                 n_launch_layers, pos, q, k, v, key_cache, val_cache, rope_cos, rope_sin, out,
                 q_norm, k_norm, norm_eps, noalloc, k_rows, v_rows, a, &W))
    return -1;
  const bool qkn = q_norm != nullptr;
  const int pf = g_sk_pf ? g_sk_pf : 2;
  // the forward pass's pending prefetch rides on this launch's spare CUs
  // (with the default two tiles in flight)
  PfLaunch pl;
  pl.n_main = (int)W;
  pl.plan = c.pf_next;
  pl.plan.per_xcd = pf_per_xcd(c.num_cus > 0 ? c.num_cus : 256, W);
  if (g_xcd_ok[c.device] != 1 || W > (c.num_cus > 0 ? c.num_cus : 256) / 4 ||
      pl.plan.per_xcd == 0 || pf != 2)
    pl.plan.n = 0;
  if (pl.plan.n > 0) {
    const dim3 pgrid((unsigned)(W + 8 * pl.plan.per_xcd)), pblock(256);
    if (head_dim == 64 && !qkn)
      hipLaunchKernelGGL((attn_decode_sk_pf_kernel<64, false>), pgrid, pblock, 0, c.stream, a, pl);
    else if (head_dim == 64)
      hipLaunchKernelGGL((attn_decode_sk_pf_kernel<64, true>), pgrid, pblock, 0, c.stream, a, pl);
    else if (!qkn)
      hipLaunchKernelGGL((attn_decode_sk_pf_kernel<128, false>), pgrid, pblock, 0, c.stream, a,
                         pl);
    else
      hipLaunchKernelGGL((attn_decode_sk_pf_kernel<128, true>), pgrid, pblock, 0, c.stream, a,
                         pl);
    return check_hip(hipGetLastError(), "attn_decode_sk_pf_kernel");
  }
  const dim3 grid((unsigned)W), block(256);
#define PLH_SK(D, Q, PF) \
  hipLaunchKernelGGL((attn_decode_sk_kernel<D, Q, PF>), grid, block, 0, c.stream, a)
  if (head_dim == 64 && !qkn) {
    if (pf == 2) PLH_SK(64, false, 2); else if (pf == 3) PLH_SK(64, false, 3); else PLH_SK(64, false, 4);
  } else if (head_dim == 64) {
    if (pf == 2) PLH_SK(64, true, 2); else if (pf == 3) PLH_SK(64, true, 3); else PLH_SK(64, true, 4);
  } else if (!qkn) {
    if (pf == 2) PLH_SK(128, false, 2); else if (pf == 3) PLH_SK(128, false, 3); else PLH_SK(128, false, 4);
  } else {
    if (pf == 2) PLH_SK(128, true, 2); else if (pf == 3) PLH_SK(128, true, 3); else PLH_SK(128, true, 4);
  }
#undef PLH_SK
  return check_hip(hipGetLastError(), "attn_decode_sk_kernel");
}

namespace plh {
bool decode_args_fused(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                       int max_seq_len, int rope_type, int layer, int pos, const float* q,
                       const float* k, const float* v, uint16_t* key_cache, uint16_t* val_cache,
                       const float* rope_cos, const float* rope_sin, float* out, DecodeArgs& a,
                       unsigned** ctr) {
  Context& c = ctx();
  if (!c.stream || !c.decode_ctr || (head_dim != 64 && head_dim != 128) || n_heads <= 0 ||
      n_kv_heads <= 0 || n_heads % n_kv_heads ||
      (rope_type != PLH_ROPE_LLAMA && rope_type != PLH_ROPE_QWEN) || max_seq_len <= 0 ||
      pos < 0 || pos >= max_seq_len || layer < 0 || layer >= n_layers || !q || !k || !v ||
      !key_cache || !val_cache || !rope_cos || !rope_sin || !out)
    return false;
  const int G = n_heads / n_kv_heads;
  const int n_groups = n_kv_heads;  // one layer, one head block per kv head
  const int npos = pos + 1;
  // the launch plh_attn_decode would queue: unsplit, the split kernel
  if (G > 16 || g_decode_kernel != 0 || npos > g_min_split ||
      use_stream_k(head_dim, pos, n_groups, c.num_cus) ||
      (long)n_groups * kFuseCtrPitch > kDecodeCounters / 2)
    return false;
  a = DecodeArgs{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.kc = key_cache;
  a.vc = val_cache;
  a.cos_t = rope_cos;
  a.sin_t = rope_sin;
  a.out = out;
  a.layer0 = layer;
  a.n_launch_layers = 1;
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.max_seq_len = max_seq_len;
  a.pos = pos;
  a.rope_type = rope_type;
  a.n_hblk = 1;
  a.nhm = G;
  a.n_split = 1;
  a.split_len = npos;
  a.n_units = n_groups;
  a.per_xcd = (n_groups + 7) / 8;
  a.G = G;
  a.fd_split = make_fastdiv(1);
  a.fd_hblk = make_fastdiv(1);
  a.fd_kvh = make_fastdiv((uint32_t)n_kv_heads);
  a.score_scale = kLog2e / sqrtf((float)head_dim);
  a.split_ctr = c.decode_ctr;
  *ctr = c.decode_ctr + kDecodeCounters / 2;  // apart from the merge counters
  return true;
}
}  // namespace plh

static int attn_decode_impl(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                            int max_seq_len, int rope_type, int layer0, int n_launch_layers,
                            int pos, const float* q, const float* k, const float* v,
                            uint16_t* key_cache, uint16_t* val_cache, const float* rope_cos,
                            const float* rope_sin, float* out, const float* q_norm,
                            const float* k_norm, float norm_eps, bool noalloc,
                            uint16_t* k_rows = nullptr, uint16_t* v_rows = nullptr) {
  Context& c = ctx();
  if (!c.stream) {
    set_error("plh_attn_decode: library not initialised");
    return -1;
  }
  if (head_dim < 2 || head_dim > 256 || head_dim % 2) {
    set_error("plh_attn_decode: head_dim %d not supported (even, at most 256)", head_dim);
    return -1;
  }
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads) {
    set_error("plh_attn_decode: n_heads %d must be a multiple of n_kv_heads %d", n_heads,
              n_kv_heads);
    return -1;
  }
  if (rope_type != PLH_ROPE_LLAMA && rope_type != PLH_ROPE_QWEN) {
    set_error("plh_attn_decode: unknown rope_type %d", rope_type);
    return -1;
  }
  if (max_seq_len <= 0 || pos < 0 || pos >= max_seq_len) {
    set_error("plh_attn_decode: pos %d outside [0, %d)", pos, max_seq_len);
    return -1;
  }
  if (layer0 < 0 || n_launch_layers <= 0 || layer0 + n_launch_layers > n_layers) {
    set_error("plh_attn_decode: layers [%d, %d) outside [0, %d)", layer0,
              layer0 + n_launch_layers, n_layers);
    return -1;
  }
  if (!q || !k || !v || !key_cache || !val_cache || !rope_cos || !rope_sin || !out) {
    set_error("plh_attn_decode: null pointer");
    return -1;
  }
  if ((q_norm == nullptr) != (k_norm == nullptr)) {
    set_error("plh_attn_decode_qknorm: q_norm and k_norm must both be given or both be null");
    return -1;
  }
  const bool qkn = q_norm != nullptr;
  if (head_dim != 64 && head_dim != 128)
    return attn_generic(n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
                        n_launch_layers, pos, 1, q, k, v, key_cache, val_cache, rope_cos,
                        rope_sin, out, n_heads * head_dim, q_norm, k_norm, norm_eps, k_rows,
                        v_rows);

  const int G = n_heads / n_kv_heads;
  const int n_hblk = (G + 15) / 16;
  const int nhm = G < 16 ? G : 16;  // q heads of the largest head block
  const int n_groups = n_launch_layers * n_kv_heads * n_hblk;
  const int npos = pos + 1;

  if (use_stream_k(head_dim, pos, n_groups, c.num_cus) && ((uintptr_t)out & 15) == 0 &&
      (long)n_groups * kSkCtrPitch <= kDecodeCounters)
    return attn_decode_sk_launch(n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
                                 n_launch_layers, pos, q, k, v, key_cache, val_cache, rope_cos,
                                 rope_sin, out, q_norm, k_norm, norm_eps, noalloc, k_rows,
                                 v_rows);

  // Split plan: contexts of at most g_min_split positions are not split (the
  // merge launch would cost more than it saves); longer ones are cut into
  // splits of a multiple of 128 rows (one 32-row tile per wave at least),
  // about `target` workgroups in all.
  const int target = g_target_units > 0 ? g_target_units : 4 * (c.num_cus > 0 ? c.num_cus : 256);
  long want_split = ((long)npos * n_groups + target - 1) / target;
  if (want_split < 128) want_split = 128;
  want_split = (want_split + 127) / 128 * 128;
  if (npos <= g_min_split) want_split = npos;
  const int split_len = (int)want_split;
  const int n_split = (npos + split_len - 1) / split_len;
  const int n_units = n_groups * n_split;
  const int groups_per_xcd = (n_groups + 7) / 8;
  const int per_xcd = groups_per_xcd * n_split;

  DecodeArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.kc = key_cache;
  a.vc = val_cache;
  a.cos_t = rope_cos;
  a.sin_t = rope_sin;
  a.out = out;
  a.part_o = a.part_m = a.part_l = nullptr;
  if (n_split > 1) {
    // per unit: (max, sum, acc[D]) of each of the block's q heads
    const size_t po = (size_t)n_units * nhm * head_dim * sizeof(float);
    const size_t pm = (size_t)n_units * nhm * sizeof(float);
    void* base;
    if (noalloc) {
      if (po + 2 * pm > kScratchBytes - kScratchCounterBytes) {
        set_error("plh_attn_decode_noalloc: this launch needs %zu bytes of split partials, "
                  "more than the %zu bytes the static scratch holds for them",
                  po + 2 * pm, kScratchBytes - kScratchCounterBytes);
        return -1;
      }
      base = (char*)g_scratch_ptr[c.device] + kScratchCounterBytes;
    } else {
      if (ensure_workspace(po + 2 * pm)) return -1;
      base = c.ws;
    }
    a.part_o = (float*)base;
    a.part_m = (float*)((char*)base + po);
    a.part_l = (float*)((char*)base + po + pm);
  }
  a.layer0 = layer0;
  a.n_launch_layers = n_launch_layers;
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.max_seq_len = max_seq_len;
  a.pos = pos;
  a.rope_type = rope_type;
  a.n_hblk = n_hblk;
  a.nhm = nhm;
  a.n_split = n_split;
  a.split_len = split_len;
  a.n_units = n_units;
  a.per_xcd = per_xcd;
  a.G = G;
  a.fd_split = make_fastdiv((uint32_t)n_split);
  a.fd_hblk = make_fastdiv((uint32_t)n_hblk);
  a.fd_kvh = make_fastdiv((uint32_t)n_kv_heads);
  a.qn = q_norm;
  a.kn = k_norm;
  a.norm_eps = norm_eps;
  a.score_scale = kLog2e / sqrtf((float)head_dim);
  a.k_rows = k_rows;
  a.v_rows = v_rows;
  // The group's last split merges in the launch when its splits share an
  // XCD (plh_init's check of the workgroup-to-XCD deal) and the counters fit
  // (tuning key 14 = -1: a combine launch instead).
  a.split_merge = n_split > 1 && g_split_merge >= 0 && g_xcd_ok[c.device] == 1 &&
                  (long)n_groups * kSplitCtrPitch <= kDecodeCounters &&
                  (size_t)n_units * nhm * head_dim * sizeof(float) < (1u << 31);
  a.split_ctr = noalloc ? (unsigned*)g_scratch_ptr[c.device] : c.decode_ctr;
  // the forward pass's pending prefetch rides on this launch's spare CUs:
  // only a launch that leaves most CUs idle takes them, one workgroup each
  PfLaunch pl;
  pl.n_main = 8 * per_xcd;
  pl.plan = c.pf_next;
  pl.plan.per_xcd = pf_per_xcd(c.num_cus > 0 ? c.num_cus : 256, 8L * per_xcd);
  if (g_xcd_ok[c.device] != 1 || 8 * per_xcd > (c.num_cus > 0 ? c.num_cus : 256) / 4 ||
      pl.plan.per_xcd == 0)
    pl.plan.n = 0;

  const dim3 grid((unsigned)(8 * per_xcd)), cblock(kCombineThreads);
  const dim3 b64(64 * DecodeShape<64>::W), b128(64 * DecodeShape<128>::W);
  if (pl.plan.n > 0) {
    const dim3 pgrid((unsigned)(8 * per_xcd + 8 * pl.plan.per_xcd));
    if (head_dim == 64 && !qkn)
      hipLaunchKernelGGL((attn_decode_pf_kernel<64, false>), pgrid, b64, 0, c.stream, a, pl);
    else if (head_dim == 64)
      hipLaunchKernelGGL((attn_decode_pf_kernel<64, true>), pgrid, b64, 0, c.stream, a, pl);
    else if (!qkn)
      hipLaunchKernelGGL((attn_decode_pf_kernel<128, false>), pgrid, b128, 0, c.stream, a, pl);
    else
      hipLaunchKernelGGL((attn_decode_pf_kernel<128, true>), pgrid, b128, 0, c.stream, a, pl);
  } else if (head_dim == 64 && !qkn) {
    hipLaunchKernelGGL((attn_decode_kernel<64, false>), grid, b64, 0, c.stream, a);
  } else if (head_dim == 64) {
    hipLaunchKernelGGL((attn_decode_kernel<64, true>), grid, b64, 0, c.stream, a);
  } else if (!qkn) {
    hipLaunchKernelGGL((attn_decode_kernel<128, false>), grid, b128, 0, c.stream, a);
  } else {
    hipLaunchKernelGGL((attn_decode_kernel<128, true>), grid, b128, 0, c.stream, a);
  }
  if (check_hip(hipGetLastError(), "attn_decode_kernel")) return -1;
  if (n_split == 1 || a.split_merge) return 0;
  // one thread per (q head of the block, d): no workgroup without work
  const int nh_max = G < 16 ? G : 16;
  const dim3 cgrid64((unsigned)(8 * groups_per_xcd),
                     (nh_max * 64 + kCombineThreads - 1) / kCombineThreads);
  const dim3 cgrid128((unsigned)(8 * groups_per_xcd),
                      (nh_max * 128 + kCombineThreads - 1) / kCombineThreads);
  const bool few = n_split <= 8;
  if (head_dim == 64 && few)
    hipLaunchKernelGGL((attn_decode_combine_kernel<64, 8>), cgrid64, cblock, 0, c.stream, a);
  else if (head_dim == 64)
    hipLaunchKernelGGL((attn_decode_combine_kernel<64, kCombineChunk>), cgrid64, cblock, 0,
                       c.stream, a);
  else if (few)
    hipLaunchKernelGGL((attn_decode_combine_kernel<128, 8>), cgrid128, cblock, 0, c.stream, a);
  else
    hipLaunchKernelGGL((attn_decode_combine_kernel<128, kCombineChunk>), cgrid128, cblock, 0,
                       c.stream, a);
  return check_hip(hipGetLastError(), "attn_decode_combine_kernel");
}

extern "C" int plh_attn_decode(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                               int max_seq_len, int rope_type, int layer0, int n_launch_layers,
                               int pos, const float* q, const float* k, const float* v,
                               uint16_t* key_cache, uint16_t* val_cache, const float* rope_cos,
                               const float* rope_sin, float* out) {
  return attn_decode_impl(n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
                          n_launch_layers, pos, q, k, v, key_cache, val_cache, rope_cos, rope_sin,
                          out, nullptr, nullptr, 0.0f, false);
}

extern "C" int plh_attn_decode_qknorm(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                                      int max_seq_len, int rope_type, int layer0,
                                      int n_launch_layers, int pos, const float* q,
                                      const float* k, const float* v, uint16_t* key_cache,
                                      uint16_t* val_cache, const float* rope_cos,
                                      const float* rope_sin, float* out, const float* q_norm,
                                      const float* k_norm, float norm_eps) {
  return attn_decode_impl(n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
                          n_launch_layers, pos, q, k, v, key_cache, val_cache, rope_cos, rope_sin,
                          out, q_norm, k_norm, norm_eps, false);
}

extern "C" int plh_attn_decode_rows(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                                    int max_seq_len, int rope_type, int layer0,
                                    int n_launch_layers, int pos, const float* q, const float* k,
                                    const float* v, uint16_t* key_cache, uint16_t* val_cache,
                                    const float* rope_cos, const float* rope_sin, float* out,
                                    const float* q_norm, const float* k_norm, float norm_eps,
                                    uint16_t* k_rows, uint16_t* v_rows) {
  if (!k_rows || !v_rows) {
    set_error("plh_attn_decode_rows: null row buffer");
    return -1;
  }
  return attn_decode_impl(n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
                          n_launch_layers, pos, q, k, v, key_cache, val_cache, rope_cos, rope_sin,
                          out, q_norm, k_norm, norm_eps, false, k_rows, v_rows);
}

extern "C" int plh_attn_decode_noalloc(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                                       int max_seq_len, int rope_type, int layer0,
                                       int n_launch_layers, int pos, const float* q,
                                       const float* k, const float* v, uint16_t* key_cache,
                                       uint16_t* val_cache, const float* rope_cos,
                                       const float* rope_sin, float* out) {
  return attn_decode_impl(n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
                          n_launch_layers, pos, q, k, v, key_cache, val_cache, rope_cos, rope_sin,
                          out, nullptr, nullptr, 0.0f, true);
}
