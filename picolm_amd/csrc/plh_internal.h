// plh_internal.h -- library-internal state and kernel argument blocks.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "fastdiv.h"
#include "l2_prefetch.h"

namespace plh {

// One device, one stream, one growable workspace: the library follows the
// reference backend's single global state (gpu.c:34-83); it is not
// re-entrant and is driven from one host thread.
struct Context {
  int device = -1;
  hipStream_t stream = nullptr;
  void* ws = nullptr;          // split-K partials
  size_t ws_bytes = 0;
  void* pf_ws = nullptr;       // prompt-chunk activations of plh_forward_prefill
  size_t pf_ws_bytes = 0;
  int num_cus = 0;
  // Arrival counters of the decode kernel's in-kernel merge (zeroed once at
  // plh_init; every launch leaves them zero).
  unsigned* decode_ctr = nullptr;
  // Workspaces outgrown by a larger call.  A graph captured before the growth
  // still holds their addresses in its kernel nodes, so every one of them
  // stays allocated until plh_shutdown (a host-side list that grows as
  // needed; both workspaces grow by 1.5x, so it stays short).
  void** retired = nullptr;
  int n_retired = 0, cap_retired = 0;
  // Operands the next decode launch warms the L2 with (set by the forward
  // pass around its attention launches; n = 0 otherwise).
  PfPlan pf_next{};
};

// Replaces the buffer *p of *bytes bytes by a new one of `want` bytes (the
// old one is retired, not freed, until plh_shutdown).  0 or -1.
int grow_buffer(void** p, size_t* bytes, size_t want, const char* what);

Context& ctx();
void set_error(const char* fmt, ...);
int check_hip(hipError_t e, const char* what);

// GEMV rows per thread forced by plh_set_tuning key 3 (0: the launch's own
// choice).
extern int g_gemv_rows_per_thread;
// plh_set_tuning key 10: 1 = the single-vector GEMVs keep the reference's x86
// AVX2 summation order bit for bit; 0 (default) = the fast order (x as int8
// digits, integer dot products), within the forward tolerance.
extern int g_gemv_exact;
// plh_set_tuning key 5: prefill chunking of small launches (0 automatic, -1
// never, 2/4/8/16 a fixed chunk size in tiles).
extern int g_prefill_split;
// plh_set_tuning key 6: prefill K-split workgroups (0 automatic, -1 never, 2
// or 3 groups of 4 waves).
extern int g_prefill_ksplit;
// plh_set_tuning key 4: 1 = the forward pass forms rmsnorm(x) in a launch of
// its own instead of inside the GEMVs that read it.
extern int g_fwd_norm_separate;

// Longest x the GEMV's rmsnorm prologue takes (its squares and the staged
// normalised x share 64 KiB of LDS).
constexpr int kGemvNormMax = 7680;

// plh_set_tuning key 15: the forward pass's attention launches warm the L2
// with the o-projection's, gate/up pair's and down projection's weights (0),
// the first two only (1), or not at all (-1).
extern int g_fwd_prefetch;
// plh_set_tuning key 17: plh_forward runs q, k, v and an unsplit attention in
// one launch, with kFusePrefetchPerXcd prefetch workgroups per XCD (0) or
// with 8..31 of them, or in two launches (-1).
extern int g_fwd_fuse;
// Prefetch workgroups per XCD of a fused q/k/v + attention launch (they share
// the CUs with its GEMV workgroups; 8, 16 and 24 measured 675, 678 and 679 us
// per TinyLlama token).
constexpr int kFusePrefetchPerXcd = 8;
// per device: 1 when workgroup c of a launch runs on XCD c % 8 (checked at
// plh_init), -1 when not, 0 before the check
extern int g_xcd_ok[64];

// One weight GEMV with the forward pass's prologue and epilogues (the
// arguments of plh_gemv_ex).
struct GemvCall {
  int qtype, n, d;
  const void* w;
  const float* x;
  float* out;
  const float* norm_w;
  float norm_eps;
  const float* bias;
  int bias_zero;
  const float* gate;
  const float* resid;
  // n_tok > 1: a batch of tokens (matmul_batch), x rows x_stride floats
  // apart and out / gate / resid rows out_stride apart; no rmsnorm prologue
  int n_tok, x_stride, out_stride;
  // with the rmsnorm prologue: also store rmsnorm(x) [n] here (or null)
  float* xn_out;
};
int gemv_launch(const GemvCall& g);
// Up to three GEMVs over the same x (and the same rmsnorm prologue, if any)
// in one launch: the q, k and v projections.
int gemv_multi_launch(const GemvCall* g, int n);
// hb = silu(gate(x)) * up(x) in one launch (model.c:906-916), gate and up of
// the same type and shape and the same rmsnorm prologue (or none); out =
// up.out.
int gemv_pair_launch(const GemvCall& gate, const GemvCall& up);
// Appends to pf the weight streams a later gemv_launch(g) (up == null) or
// gemv_pair_launch(g, *up) reads, chunked as its workgroups read them; -1
// (pf unchanged) when the call is not a single-vector GEMV or pf is full.
int gemv_prefetch_plan(const GemvCall& g, const GemvCall* up, PfPlan& pf);

// Looks up (once per device, with that device current) the device address of
// the decode kernels' static scratch array; plh_init calls it.  0 or -1.
int decode_scratch_setup(int device);

// Makes sure the workspace holds at least `bytes` (the outgrown one is
// retired until plh_shutdown).  Returns 0 or -1.
int ensure_workspace(size_t bytes);
// Capacity of Context::decode_ctr and of the static scratch's counter region,
// in counters; the stream-K kernel keeps one per 32 (a 128-byte line), so a
// launch of at most kDecodeCounters / 32 (layer, kv head, q-head block)
// groups runs it.
constexpr int kDecodeCounters = 1 << 18;

// Attention of the head dims without a tuned kernel (every even head_dim up
// to 256 but 64 and 128; attn_generic.hip): append and attend n_tokens rows
// at start_pos.. of layers layer0.. (decode: n_tokens 1, out_stride
// n_heads*head_dim).  Arguments are checked by the caller.  0 or -1.
int attn_generic(int n_heads, int n_kv_heads, int head_dim, int max_seq_len, int rope_type,
                 int layer0, int n_launch_layers, int start_pos, int n_tokens, const float* q,
                 const float* k, const float* v, uint16_t* key_cache, uint16_t* val_cache,
                 const float* rope_cos, const float* rope_sin, float* out, int out_stride,
                 const float* q_norm, const float* k_norm, float norm_eps, uint16_t* k_rows,
                 uint16_t* v_rows);

// Decode kernel arguments (all device pointers).
struct DecodeArgs {
  const float* q;          // [n_launch_layers][n_heads*D]
  const float* k;          // [n_launch_layers][kv_dim]
  const float* v;          // [n_launch_layers][kv_dim]
  uint16_t* kc;            // [n_layers][S][kv_dim] fp16 bits
  uint16_t* vc;
  const float* cos_t;      // [S][D/2]
  const float* sin_t;
  float* out;              // [n_launch_layers][n_heads*D]
  float* part_o;           // [n_units][nhm][D]
  float* part_m;           // [n_units][nhm]
  float* part_l;           // [n_units][nhm]
  int layer0, n_launch_layers, n_heads, n_kv_heads, max_seq_len, pos, rope_type;
  int n_hblk;              // ceil(G / 16): q-head blocks per kv head
  int nhm;                 // min(G, 16): partial slots per unit
  int n_split, split_len;  // position splits per (layer, kv head, head block)
  int n_units;             // n_groups * n_split
  int per_xcd;             // units per XCD slice of the grid
  const float* qn;         // QK-norm weights [n_launch_layers][D], or null
  const float* kn;
  float norm_eps;
  float score_scale;       // log2(e) / sqrt(D)
  uint16_t* k_rows;        // the appended rows also here [n_launch_layers][kv_dim], or null
  uint16_t* v_rows;
  // Stream-K plan (attn_decode_sk_kernel): the groups' cached rows in 16-row
  // blocks, flattened group-major (sk_nbk blocks per group) and cut into one
  // range per workgroup, ranges of sk_q or sk_q + 1 blocks (the first sk_r
  // take sk_q + 1).  A group covered by several
  // ranges is merged in the kernel by its last-arriving producer through
  // sk_part (sk_maxp slots per group of nhm x (D + 4) floats) and the
  // self-resetting arrival counters sk_ctr (one per group, zero between
  // launches).
  int sk_q, sk_r, sk_nbk, sk_maxp, sk_groups;
  float* sk_part;
  uint32_t sk_part_bytes;
  unsigned* sk_ctr;
  // n_heads / n_kv_heads, and divisions by the launch's constants
  int G;
  FastDiv fd_split, fd_hblk, fd_kvh;  // n_split, n_hblk, n_kv_heads
  FastDiv fd_nbk, fd_q, fd_q1;         // sk_nbk, sk_q, sk_q + 1
  // split kernel: a group's last split to finish merges the partials itself
  // (through its XCD's L2, counting on split_ctr) instead of a combine launch
  int split_merge;
  unsigned* split_ctr;
  // stream-K ranges per XCD (0: ranges in workgroup order) and its division
  int sk_wx;
  FastDiv fd_wx;
  // sk_k > 0: W = sk_k * n_groups ranges, sk_k (a power of two, 1 << sk_kshift,
  // at most sk_nbk) to a group, each group's blocks split evenly among its own
  // (else the flattened blocks cut into W ranges)
  int sk_k, sk_kshift;
};

// The fused q/k/v + attention launch of plh_forward (short contexts): the
// arguments of the unsplit one-layer decode launch plh_attn_decode would
// queue for this call, and the counters the attention workgroups wait on;
// false (nothing set) when that call would take another kernel or split.
bool decode_args_fused(int n_layers, int n_heads, int n_kv_heads, int head_dim,
                       int max_seq_len, int rope_type, int layer, int pos, const float* q,
                       const float* k, const float* v, uint16_t* key_cache, uint16_t* val_cache,
                       const float* rope_cos, const float* rope_sin, float* out, DecodeArgs& a,
                       unsigned** ctr);
// q, k and v (g[0..2], the rmsnorm prologue, fast order) and the attention of
// d in one launch: d's groups' attention workgroups first, then the q/k/v
// GEMV workgroups, which count themselves in on ctr, then pf_per_xcd
// workgroups per XCD prefetching pf (none when pf.n is 0).  -1 on error.
int qkv_attention_launch(const GemvCall* g, const DecodeArgs& d, int head_dim, unsigned* ctr,
                         const PfPlan& pf, int pf_per_xcd);

}  // namespace plh

namespace plh {

// Prefill kernel arguments (all device pointers).
struct PrefillArgs {
  const float* q;          // [n_launch_layers][n_tokens][n_heads*D]
  const float* k;          // [n_launch_layers][n_tokens][kv_dim]
  const float* v;          // [n_launch_layers][n_tokens][kv_dim]
  uint16_t* kc;            // [n_layers][S][kv_dim] fp16 bits
  uint16_t* vc;
  const float* cos_t;      // [S][D/2]
  const float* sin_t;
  float* out;              // [n_launch_layers][n_tokens][out_stride]
  int layer0, n_launch_layers, n_heads, n_kv_heads, max_seq_len, rope_type;
  int start_pos, n_tokens, out_stride;
  int bq;                  // tokens per q block
  int n_qblk;              // q blocks per (layer, kv head)
  int n_units;             // n_launch_layers * n_kv_heads * n_qblk
  int per_xcd;             // workgroups per XCD slice of the grid
  int xcd_slices;          // 8 (block b runs on XCD b % 8 and takes slice b % 8) or 1
  int groups_per_xcd;      // (layer, kv head) groups per slice
  int qb_major;            // single blocks: order a slice's units by q block, heaviest first
  int paired;              // 1: a workgroup runs a heavy q block and its light mirror
  int split_tiles;         // > 0: units split into chunks of this many tiles
  int chunks_per_group;    // chunks of one (layer, kv head) group when split
  float* part_o;           // split partials [n_groups*chunks_per_group][128 columns][D]
  float* part_m;           // [..][128] running maxima (log2 units)
  float* part_l;           // [..][128] running sums
  const float* qn;         // QK-norm weights [n_launch_layers][D], or null
  const float* kn;
  float norm_eps;
  float score_scale;       // log2(e) / sqrt(D)
  // the append's item decomposition: division by n_kv_heads and n_tokens
  // (items fit 32 bits when app32 is set)
  int app32;
  FastDiv fd_app_kvh, fd_app_tok;
};

}  // namespace plh
