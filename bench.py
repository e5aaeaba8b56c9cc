"""Benchmark of picolm's attention block on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one token's decode attention over all layers of the model (one
plh_attn_decode call covering every layer), with inputs resident in HBM.
The default workload is TinyLlama-1.1B-shaped decode at position 2047
(22 layers, 32 q heads, 4 kv heads, head_dim 64, FP16 cache of 2048 rows);
the same line carries, under "prefill", the TinyLlama-shaped 512-token causal
prefill (all 22 layers per step) in TFLOP/s of causal-pair flops
(L * Hq * 4D * sum_i (i+1)) against its binding roof (HBM, for the fp32
q/k/v/out traffic at these sizes), with the fraction of the fp16 MFMA peak.

Method:
  * the FP16 caches are rotated over enough copies (>= 512 MiB in total) that
    the 256 MiB Infinity Cache cannot serve a step from the previous one;
  * the K timed steps are captured into one HIP graph (no host launch cost
    between steps); the graph is replayed once untimed and once timed,
    bracketed by device synchronisation.  ms_per_step is the wall clock of the
    timed replay / K; roofline.achieved uses hipEvents recorded on the library
    stream around the timed replay (mean duration per launch);
  * algorithmic bytes per token (all layers):
      L * [ (pos+1)*2*Hkv*D*2  (K+V rows read)
            + Hq*D*4 + 2*Hkv*D*4 (q, k, v in) + 2*Hkv*D*2 (row written)
            + Hq*D*4 (out) ]
  * per_layer_launches: the same token as L sequential one-layer calls (how
    a per-layer forward pass uses the block), also graph-replayed;
  * cpu_baseline: the reference's own decode attention where oracle/_ref (its
    sources compiled) exists: its model_forward at position pos minus the same
    token at position 0, on the forward workload's model (same attention
    shape), matmuls on the host threads -- the reference runs its attention
    loop on one thread whatever its -j; cpu_baseline_port (or cpu_baseline
    without oracle/_ref or with --no-forward): the oracle (the attention
    restated in C, same op order, out-of-line fp16 widening as in the
    reference build) on one host thread over a bounded sample;
    cpu_baseline_head_parallel: the same arithmetic with the q heads split
    over up to 16 host threads, an upper bound only; "host" records nproc,
    the CPU model and the C library;
  * gemv: every weight GEMV of one TinyLlama Q4_K_M-style token (the
    gpu_try_matmul path: 22 x (q, k, v, o, gate, up, down) + output, 670 MB
    of GGUF weights), graph-replayed, against the HBM roof; its CPU baseline
    is the oracle matmul with rows split over the host threads like the
    reference's matmul pool, and the sampled GPU outputs are checked bit for
    bit against it;
  * forward: the whole forward pass on the device (plh_forward) for a
    TinyLlama-shaped Q4_K_M-style synthetic model: prefill of a 128-token
    prompt, decode tok/s (tokens queued back to back) and greedy-generation
    tok/s (logits to the host and argmax every token); its CPU baseline is
    the reference's own model_forward compiled from its sources
    (oracle/_ref, the oracle forward pass where that library is absent) on
    the host threads, and the GPU logits of the sampled tokens are checked
    against it.
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "attn µs/token + KV GB/s (% HBM peak) decode; prefill TFLOP/s (% MFMA)"
HBM_PEAK_GBS = 8000.0
MALL_DEFEAT_BYTES = 512 << 20

MFMA_F16_PEAK_TFS = 2516.6

HOST_THREADS_MAX = 16   # host CPU threads available per GPU

WORKLOADS = {
    "tinyllama_decode_pos2047": dict(L=22, Hq=32, Hkv=4, D=64, S=2048, theta=1e4, pos=2047),
    "tinyllama_decode_pos256": dict(L=22, Hq=32, Hkv=4, D=64, S=2048, theta=1e4, pos=256),
    "llama32_decode_pos8191": dict(L=16, Hq=32, Hkv=8, D=64, S=8192, theta=5e5, pos=8191),
    "llama2_decode_pos4095": dict(L=32, Hq=32, Hkv=32, D=128, S=4096, theta=1e4, pos=4095),
    "tinyllama_prefill_512": dict(L=22, Hq=32, Hkv=4, D=64, S=2048, theta=1e4, start=0, n=512),
    "llama2_prefill_1024": dict(L=32, Hq=32, Hkv=32, D=128, S=4096, theta=1e4, start=0, n=1024),
    # Qwen3-0.6B-shaped: half-split rotation and per-head QK-norm (eps 1e-6)
    "qwen3_decode_pos2047": dict(L=28, Hq=16, Hkv=8, D=128, S=2048, theta=1e6, pos=2047, rt=1,
                                 qkn=1e-6),
    "qwen3_prefill_512": dict(L=28, Hq=16, Hkv=8, D=128, S=2048, theta=1e6, start=0, n=512,
                              rt=1, qkn=1e-6),
}


# The weight GEMVs of one token of a TinyLlama-1.1B Q4_K_M-style model (the
# matmuls picolm hands to gpu_try_matmul): per layer q, k, v, o, gate, up,
# down (v and down Q6_K, the rest Q4_K), then the Q6_K output projection.
GEMV_TOKEN = dict(L=22, n_embd=2048, n_ffn=5632, kv_dim=256, vocab=32000)
GEMV_WORKLOAD = "tinyllama_q4km_gemv_token"
Q4K, Q6K = 12, 14


def gemv_matrices(g=GEMV_TOKEN):
    """(qtype, n, d) of every GEMV of one token, in forward-pass order."""
    e, f, kv = g["n_embd"], g["n_ffn"], g["kv_dim"]
    layer = [(Q4K, e, e), (Q4K, e, kv), (Q6K, e, kv), (Q4K, e, e), (Q4K, e, f), (Q4K, e, f),
             (Q6K, f, e)]
    return layer * g["L"] + [(Q6K, e, g["vocab"])]


def gemv_bytes(mats) -> int:
    """GGUF weight bytes + fp32 x in + fp32 out, per token."""
    total = 0
    for qt, n, d in mats:
        rb = n // 256 * (144 if qt == Q4K else 210)
        total += d * rb + n * 4 + d * 4
    return total


def run_gemv(P, steps, warmup):
    """One step = every weight GEMV of one token (155 launches, device
    pointers, graph-replayed); the 670 MB of weights exceed the Infinity
    Cache, so each step streams them from HBM."""
    from picolm_amd import gemv as G
    from picolm_amd import synth as S
    mats = gemv_matrices()
    rng = np.random.default_rng(155)
    host = {}
    for key in sorted(set(mats)):   # one random matrix per shape, one device copy per use
        host[key] = S.random_weights(rng, *(key[0], key[1], key[2]))
    dev, xs, outs = [], [], []
    for qt, n, d in mats:
        dev.append(G.QMatrix(qt, n, d, host[(qt, n, d)]))
        xs.append(P.DeviceBuffer.from_numpy(rng.standard_normal(n).astype(np.float32)))
        outs.append(P.DeviceBuffer(d * 4))
    P.synchronize()

    def launch():
        for W, x, o in zip(dev, xs, outs):
            G.matmul(o.ptr, x.ptr, W)

    for _ in range(max(1, warmup)):
        launch()
    P.synchronize()
    with P.Graph() as g:
        for _ in range(steps):
            launch()
    g.launch()
    P.synchronize()
    e0, e1 = P.Event(), P.Event()
    t0 = time.perf_counter()
    e0.record()
    g.launch()
    e1.record()
    P.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1) / steps
    algo = gemv_bytes(mats)
    achieved = algo / (ms * 1e-3) / 1e9
    return {
        "us_per_token": wall * 1e6 / steps,
        "gbs": algo / (wall / steps) / 1e9,
        "launches_per_token": len(mats),
        "algorithmic_bytes_per_step": algo,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None},
        "_inputs": (mats, host, xs, outs),
    }


def cpu_baseline_gemv(res, budget_s=8.0):
    """The oracle's matmul (bit-identical to the reference's x86-64 AVX2
    vec_dot) on the host's cores, rows split over threads like the
    reference's matmul pool, over a bounded sample of the token's GEMVs;
    with a bit-exact check of the GPU outputs of the sampled GEMVs."""
    from oracle import oracle as O
    mats, host, xs, outs = res.pop("_inputs")
    n_thr = min(os.cpu_count() or 1, HOST_THREADS_MAX)
    t_total, done_bytes, checked, exact = 0.0, 0, 0, True
    for i, (qt, n, d) in enumerate(mats):
        if t_total >= budget_s:
            break
        x = xs[i].download(np.float32, (n,))
        W = host[(qt, n, d)]
        t0 = time.perf_counter()
        ref = O.matmul_mt(W, x, n, d, qt, n_thr)
        t_total += time.perf_counter() - t0
        done_bytes += d * (n // 256) * (144 if qt == Q4K else 210) + n * 4 + d * 4
        got = outs[i].download(np.float32, (d,))
        exact = exact and bool(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))
        checked += 1
    return {"cpu_baseline": {"value": done_bytes / t_total / 1e9, "unit": "GB/s",
                             "cores": n_thr, "kind": "port",
                             "us_per_token": t_total / done_bytes * gemv_bytes(mats) * 1e6,
                             "sample": f"the first {checked} of {len(mats)} GEMVs of the token, "
                                       f"oracle rows split over {n_thr} threads"},
            "parity_bit_exact_sampled": exact, "parity_gemvs_checked": checked}


# The whole forward pass (model_forward on the device, plh_forward): a
# TinyLlama-1.1B-shaped Q4_K_M-style synthetic model (Q4_K embedding, q, k,
# o, gate, up; Q6_K v, down, output).
FWD_MODEL = dict(n_layers=22, n_embd=2048, n_ffn=5632, n_heads=32, n_kv_heads=4, head_dim=64,
                 vocab_size=32000, max_seq_len=2048)
FWD_WORKLOAD = "tinyllama_q4km_forward"


def run_forward(P, n_prompt=128, n_decode=64, n_check=8):
    """Prefill of an n_prompt-token prompt (plh_forward_prefill), then two
    decode loops from position n_prompt: `decode` queues n_decode tokens
    back to back (token ids fixed in advance, device time per token), and
    `generate` is greedy generation as picolm's loop runs it: every token's
    logits copied to the host, argmax, the next call (host round trip
    included).  The first n_check tokens of the prompt are also run as
    decode steps from position 0 and kept for the CPU leg's parity check."""
    from picolm_amd import synth as S
    t0 = time.perf_counter()
    h = S.SynthModel(**FWD_MODEL, seed=7, share_layers=True)
    dm = P.DeviceModel(h)
    P.synchronize()
    setup_s = time.perf_counter() - t0
    rng = np.random.default_rng(8)
    prompt = rng.integers(0, h.vocab_size, n_prompt).astype(np.int32)
    check = []
    for i in range(n_check):
        dm.forward(int(prompt[i]), i)
        P.synchronize()
        check.append(dm.fetch_logits())
    # prefill over the whole prompt (rows 0..n_check-1 are rewritten)
    dm.prefill(prompt, 0)
    P.synchronize()
    t0 = time.perf_counter()
    dm.prefill(prompt, 0)
    P.synchronize()
    prefill_s = time.perf_counter() - t0
    toks = rng.integers(0, h.vocab_size, n_decode + 4)
    for i in range(4):
        dm.forward(int(toks[i]), n_prompt + i)
    P.synchronize()
    e0, e1 = P.Event(), P.Event()
    t0 = time.perf_counter()
    e0.record()
    for i in range(n_decode):
        dm.forward(int(toks[4 + i]), n_prompt + 4 + i)
    e1.record()
    P.synchronize()
    wall = (time.perf_counter() - t0) / n_decode
    dev_ms = e0.elapsed_ms(e1) / n_decode
    pos = n_prompt + 4 + n_decode
    tok = int(toks[-1])
    t0 = time.perf_counter()
    for i in range(n_decode):
        dm.forward(tok, pos + i)
        tok = int(np.argmax(dm.fetch_logits()))
    gen = (time.perf_counter() - t0) / n_decode
    wb = h.weight_bytes_per_token()
    gbs = wb / (dev_ms * 1e-3) / 1e9
    res = {
        "workload": FWD_WORKLOAD,
        "config": dict(FWD_MODEL, types="Q4_K embd/q/k/o/gate/up, Q6_K v/down/output",
                       prompt=n_prompt),
        "decode_tok_s": 1.0 / wall,
        "decode_us_per_token": wall * 1e6,
        "decode_device_us_per_token": dev_ms * 1e3,
        "generate_tok_s": 1.0 / gen,
        "generate_us_per_token": gen * 1e6,
        "prefill_tok_s": n_prompt / prefill_s,
        "prefill_ms": prefill_s * 1e3,
        "weight_bytes_per_token": wb,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None,
                     "note": "GGUF weight bytes per token / device time per decode token"},
        "setup_s": setup_s,
        "_check": (h, prompt[:n_check], check),
    }
    dm.free()
    return res


def cpu_baseline_forward(res):
    """picolm's own model_forward (the reference's model.c / tensor.c /
    quant.c compiled from its sources into oracle/_ref, AVX2 build, its
    matmul thread pool at the host's threads) on the first tokens of the
    prompt from position 0; without that library the oracle's forward pass
    (bit-identical to it) stands in.  The GPU logits of the same steps are
    checked against the CPU's (normwise, the attention/silu exp tolerance)
    with the greedy token."""
    from oracle import oracle as O
    h, toks, gpu_logits = res.pop("_check")
    n_thr = min(os.cpu_count() or 1, HOST_THREADS_MAX)
    if O.ref_available():
        O.ref().ref_set_threads(n_thr)
        cpu, kind, what = O.RefForward(h), "reference", "picolm model_forward (oracle/_ref)"
        step = cpu.forward
    else:
        cpu, kind, what = O.OracleForward(h), "port", "oracle model_forward"
        step = lambda t, p: cpu.forward(t, p, n_threads=n_thr)   # noqa: E731
    worst, same_argmax, t_total = 0.0, True, 0.0
    for i, t in enumerate(toks):
        t0 = time.perf_counter()
        lo, _ = step(int(t), i)
        t_total += time.perf_counter() - t0
        g = gpu_logits[i]
        worst = max(worst, float(np.max(np.abs(g - lo)) / np.max(np.abs(lo))))
        same_argmax = same_argmax and int(np.argmax(g)) == int(np.argmax(lo))
    if kind == "reference":
        O.ref().ref_set_threads(1)
        cpu.close()
    return {"cpu_baseline": {"value": len(toks) / t_total, "unit": "tok/s", "cores": n_thr,
                             "kind": kind,
                             "sample": f"{what} of the first {len(toks)} prompt tokens "
                                       f"(positions 0..{len(toks) - 1}), {n_thr} matmul threads"},
            "parity_logits_normwise_max": worst, "parity_greedy_token_same": same_argmax}


def cpu_reference_attention(h, w, reps=3):
    """The reference's own decode attention (model.c:828-892) timed inside its
    model_forward (oracle/_ref): the same TinyLlama-shaped model run at
    position pos over rows 0..pos-1 of N(0,1) fp16 cache rows, minus the same
    token at position 0 (everything but the attention loop costs the same at
    both positions).  The matmuls use the host threads; the attention loop
    runs on one thread whatever -j is (model.c:848-892).  None without
    oracle/_ref or when the model's attention shape is not the workload's."""
    from oracle import oracle as O
    if not O.ref_available():
        return None
    if (h.n_layers, h.n_heads, h.n_kv_heads, h.head_dim, h.max_seq_len) != (
            w["L"], w["Hq"], w["Hkv"], w["D"], w["S"]) or h.rope_type != w.get("rt", 0):
        return None
    pos = w["pos"]
    n_thr = min(os.cpu_count() or 1, HOST_THREADS_MAX)
    O.ref().ref_set_threads(n_thr)
    ref = O.RefForward(h)
    try:
        rng = np.random.default_rng(2047)
        kv = h.n_kv_heads * h.head_dim
        for cache in (ref.kc, ref.vc):
            view = cache.reshape(h.n_layers, h.max_seq_len, kv)
            for layer in range(h.n_layers):
                view[layer, :pos] = O.f32_to_f16(
                    rng.standard_normal((pos, kv), dtype=np.float32)).reshape(pos, kv)
        ref.forward(1, pos)                       # warm-up (writes row pos only)
        t_long, t_short = [], []
        for _ in range(reps):
            t0 = time.perf_counter()
            ref.forward(1, pos)
            t_long.append(time.perf_counter() - t0)
            t0 = time.perf_counter()
            ref.forward(1, 0)
            t_short.append(time.perf_counter() - t0)
    finally:
        O.ref().ref_set_threads(1)
        ref.close()
    attn_s = float(np.median(t_long) - np.median(t_short))
    return {"value": decode_bytes(w) / attn_s / 1e9, "unit": "GB/s", "cores": 1,
            "kind": "reference", "us_per_token": attn_s * 1e6,
            "sample": f"picolm model_forward (oracle/_ref) at pos {pos} minus pos 0, {reps} "
                      f"runs each, on the forward workload's model (same attention shape); "
                      f"matmuls on {n_thr} threads, the attention loop on one"}


def qkn_bytes(w) -> int:
    """The q and k norm weight rows read per launch (all layers), if any."""
    return w["L"] * 2 * w["D"] * 4 if w.get("qkn") else 0


def decode_bytes(w) -> int:
    L, Hq, Hkv, D, pos = w["L"], w["Hq"], w["Hkv"], w["D"], w["pos"]
    per_layer = ((pos + 1) * 2 * Hkv * D * 2 + Hq * D * 4 + 2 * Hkv * D * 4
                 + 2 * Hkv * D * 2 + Hq * D * 4)
    return L * per_layer + qkn_bytes(w)


def prefill_flops(w) -> int:
    """Causal pairs only: L * Hq * 4D * sum_{i<N} (start + i + 1)."""
    n, st = w["n"], w["start"]
    pairs = n * st + n * (n + 1) // 2
    return w["L"] * w["Hq"] * 4 * w["D"] * pairs


def prefill_bytes(w) -> int:
    """fp32 q, k, v in and out, fp16 rows appended, per launch (all layers)."""
    L, n, Hq, Hkv, D = w["L"], w["n"], w["Hq"], w["Hkv"], w["D"]
    return L * n * (Hq * D * 4 * 2 + 2 * Hkv * D * 4 + 2 * Hkv * D * 2) + qkn_bytes(w)


def traffic_from_profiles(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated against a copy kernel), if a summary exists."""
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes")
    except (OSError, ValueError):
        return None


def norm_weights(P, w, rng):
    """Device [L][D] q and k norm weights for a QK-norm workload, else None."""
    if not w.get("qkn"):
        return None, None
    shape = (w["L"], w["D"])
    qn = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
    kn = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
    return P.DeviceBuffer.from_numpy(qn), P.DeviceBuffer.from_numpy(kn)


def run_decode(P, w, steps, warmup, name):
    rt = w.get("rt", 0)
    cfg = P.AttnConfig(w["L"], w["Hq"], w["Hkv"], w["D"], w["S"], w["theta"], rt)
    cache_bytes = cfg.cache_elems * 2
    n_copies = max(1, math.ceil(MALL_DEFEAT_BYTES / (2 * cache_bytes)))
    rng = np.random.default_rng(2047)
    pos = w["pos"]

    # copy 0: rows 0..pos-1 of every layer hold N(0,1) rounded to fp16 on the
    # device with the reference's rounding; other rows are zero
    L, S, kv = cfg.n_layers, cfg.max_seq_len, cfg.kv_dim
    cos_t, sin_t = P.rope_tables(S, cfg.head_dim, cfg.rope_freq_base)
    d_cos, d_sin = P.DeviceBuffer.from_numpy(cos_t), P.DeviceBuffer.from_numpy(sin_t)
    staging = P.DeviceBuffer(L * S * kv * 4)
    keys, vals = [], []
    for which in range(2):
        host = np.zeros((L, S, kv), np.float32)
        host[:, :pos] = rng.standard_normal((L, pos, kv), dtype=np.float32)
        staging.upload(host)
        buf = P.DeviceBuffer(cache_bytes)
        P.f32_to_f16(staging.ptr, buf.ptr, L * S * kv)
        (keys if which == 0 else vals).append(buf)
        del host
    staging.free()
    for c in range(1, n_copies):
        for lst in (keys, vals):
            b = P.DeviceBuffer(cache_bytes)
            b.copy_from(lst[0])
            lst.append(b)
    qkv = []
    for c in range(n_copies):
        q = P.DeviceBuffer.from_numpy(rng.standard_normal((L, cfg.q_dim), dtype=np.float32))
        k = P.DeviceBuffer.from_numpy(rng.standard_normal((L, kv), dtype=np.float32))
        v = P.DeviceBuffer.from_numpy(rng.standard_normal((L, kv), dtype=np.float32))
        o = P.DeviceBuffer(L * cfg.q_dim * 4)
        qkv.append((q, k, v, o))
    d_qn, d_kn = norm_weights(P, w, rng)
    P.synchronize()

    def call(layer0, n_layers, q, k, v, c, o):
        """One plh_attn_decode(_qknorm) call over layers layer0.. (pointers
        already offset to layer0)."""
        common = (L, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, S, rt, layer0, n_layers, pos,
                  q, k, v, keys[c].ptr, vals[c].ptr, d_cos.ptr, d_sin.ptr, o)
        if d_qn is None:
            P.check(P.lib.plh_attn_decode(*common), "plh_attn_decode")
        else:
            off = layer0 * cfg.head_dim * 4
            P.check(P.lib.plh_attn_decode_qknorm(*common, d_qn.ptr + off, d_kn.ptr + off,
                                                 w["qkn"]), "plh_attn_decode_qknorm")

    def launch(i):
        c = i % n_copies
        q, k, v, o = qkv[c]
        call(0, L, q.ptr, k.ptr, v.ptr, c, o.ptr)

    for i in range(max(1, warmup)):   # also sizes the split-K workspace
        launch(i)
    P.synchronize()

    with P.Graph() as g:
        for i in range(steps):
            launch(i)
    g.launch()                     # untimed replay
    P.synchronize()
    e0, e1 = P.Event(), P.Event()
    t0 = time.perf_counter()
    e0.record()
    g.launch()
    e1.record()
    P.synchronize()
    wall = time.perf_counter() - t0
    k_mean = e0.elapsed_ms(e1) / steps

    # the same token as L sequential one-layer launches (how a per-layer
    # forward pass calls the block), timed the same way over fewer steps
    pl_steps = max(1, steps // 10)
    def launch_per_layer(i):
        c = i % n_copies
        q, k, v, o = qkv[c]
        for l in range(L):
            call(l, 1, q.ptr + l * cfg.q_dim * 4, k.ptr + l * kv * 4, v.ptr + l * kv * 4, c,
                 o.ptr + l * cfg.q_dim * 4)
    launch_per_layer(0)
    P.synchronize()
    with P.Graph() as g2:
        for i in range(pl_steps):
            launch_per_layer(i)
    g2.launch()
    P.synchronize()
    e0.record()
    g2.launch()
    e1.record()
    P.synchronize()
    pl_ms = e0.elapsed_ms(e1) / pl_steps

    # warm: every step reuses copy 0, so a cache that fits the 256 MiB
    # Infinity Cache is served from it (reported apart, never the headline)
    def launch_warm(i):
        q, k, v, o = qkv[0]
        call(0, L, q.ptr, k.ptr, v.ptr, 0, o.ptr)
    with P.Graph() as g3:
        for i in range(steps):
            launch_warm(i)
    g3.launch()
    P.synchronize()
    e0.record()
    g3.launch()
    e1.record()
    P.synchronize()
    warm_ms = e0.elapsed_ms(e1) / steps

    algo = decode_bytes(w)
    ms_step = wall * 1e3 / steps
    achieved = algo / (k_mean * 1e-3) / 1e9
    result = {
        "value": algo / (ms_step * 1e-3) / 1e9,
        "unit": "GB/s",
        "ms_per_step": ms_step,
        "us_per_token": ms_step * 1e3,
        "kernel_us_mean": k_mean * 1e3,
        "algorithmic_bytes_per_step": algo,
        "cache_copies_rotated": n_copies,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic_from_profiles(name)},
        "per_layer_launches": {"us_per_token": pl_ms * 1e3,
                               "gbs": algo / (pl_ms * 1e-3) / 1e9,
                               "launches_per_token": L},
        "warm": {"us_per_token": warm_ms * 1e3,
                 "gbs": algo / (warm_ms * 1e-3) / 1e9,
                 "note": "one cache copy reused every step: Infinity-Cache resident when "
                         "it fits in 256 MiB; not the headline"},
    }
    # keep what the CPU baseline needs (copy 0 before further appends)
    result["_cpu_inputs"] = (cfg, keys[0], vals[0], qkv[0], cos_t, sin_t, d_qn, d_kn)
    return result


def run_prefill(P, w, steps, warmup):
    """One step = prefill of n prompt tokens over all layers (append kernel +
    causal attention kernel), inputs rotated over enough copies to defeat the
    Infinity Cache."""
    cfg = P.AttnConfig(w["L"], w["Hq"], w["Hkv"], w["D"], w["S"], w["theta"], w.get("rt", 0))
    L, n, st = cfg.n_layers, w["n"], w["start"]
    per_copy = prefill_bytes(w) + 2 * L * n * cfg.kv_dim * 2
    n_copies = max(2, math.ceil(MALL_DEFEAT_BYTES / per_copy))
    rng = np.random.default_rng(512)
    copies = []
    for c in range(n_copies):
        cache = P.KVCache(cfg)
        q = P.DeviceBuffer.from_numpy(rng.standard_normal((L, n, cfg.q_dim), dtype=np.float32))
        k = P.DeviceBuffer.from_numpy(rng.standard_normal((L, n, cfg.kv_dim), dtype=np.float32))
        v = P.DeviceBuffer.from_numpy(rng.standard_normal((L, n, cfg.kv_dim), dtype=np.float32))
        o = P.DeviceBuffer(L * n * cfg.q_dim * 4)
        copies.append((cache, q, k, v, o))
    d_qn, d_kn = norm_weights(P, w, rng)
    norms = {} if d_qn is None else dict(q_norm=d_qn.ptr, k_norm=d_kn.ptr, norm_eps=w["qkn"])
    P.synchronize()

    def launch(i):
        cache, q, k, v, o = copies[i % n_copies]
        P.prefill(cache, 0, st, n, q.ptr, k.ptr, v.ptr, o.ptr, None, L, **norms)

    for i in range(max(1, warmup)):
        launch(i)
    P.synchronize()
    with P.Graph() as g:
        for i in range(steps):
            launch(i)
    g.launch()
    P.synchronize()
    e0, e1 = P.Event(), P.Event()
    t0 = time.perf_counter()
    e0.record()
    g.launch()
    e1.record()
    P.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1) / steps
    flops = prefill_flops(w)
    algo_bytes = prefill_bytes(w)
    tfs = flops / (ms * 1e-3) / 1e12
    # the binding roof at this arithmetic intensity: HBM (expressed in TFLOP/s)
    # below the fp16 ridge, else the MFMA peak; MFMA utilisation beside it
    hbm_roof = flops / algo_bytes * HBM_PEAK_GBS / 1e3
    roof = min(MFMA_F16_PEAK_TFS, hbm_roof)
    return {
        "us_per_step": wall * 1e6 / steps,
        "us_per_token": wall * 1e6 / steps / n,
        "tflops": tfs,
        "roofline": {"bound": "hbm" if hbm_roof < MFMA_F16_PEAK_TFS else "mfma",
                     "achieved": tfs, "peak": roof, "unit": "TFLOP/s", "frac": tfs / roof,
                     "achieved_gbs": algo_bytes / (ms * 1e-3) / 1e9,
                     "mfma_peak": MFMA_F16_PEAK_TFS, "mfma_frac": tfs / MFMA_F16_PEAK_TFS},
        "algorithmic_flops_per_step": flops,
        "algorithmic_bytes_per_step": algo_bytes,
        "copies_rotated": n_copies,
        "_copies": copies,
        "_norms": (d_qn, d_kn),
    }


def cpu_baseline_prefill(P, w, res, budget_s=8.0):
    """The oracle's prefill on one host thread over a bounded number of layers
    of the same step, extrapolated to all layers."""
    from oracle import oracle as O
    cache, dq, dk, dv, dout = res.pop("_copies")[0]
    cfg = cache.cfg
    L, n, st = cfg.n_layers, w["n"], w["start"]
    kc, vc = cache.fetch()
    shp = O.Shape(L, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
                  cfg.rope_freq_base, cfg.rope_type)
    qn, kn = host_norms(res.pop("_norms"), L, cfg.head_dim)
    cos_t, sin_t = O.rope_tables(cfg.max_seq_len, cfg.head_dim, cfg.rope_freq_base)
    q = dq.download(np.float32, (L, n, cfg.q_dim))
    k = dk.download(np.float32, (L, n, cfg.kv_dim))
    v = dv.download(np.float32, (L, n, cfg.kv_dim))
    gpu_out = dout.download(np.float32, (L, n, cfg.q_dim))
    t_total, layers, worst = 0.0, 0, 0.0
    while t_total < budget_s and layers < L:
        t0 = time.perf_counter()
        ref = O.attn_prefill(shp, layers, st, n, q[layers].copy(), k[layers].copy(), v[layers],
                             kc, vc, cos_t, sin_t, **norm_args(w, qn, kn, layers))
        t_total += time.perf_counter() - t0
        err = np.abs(gpu_out[layers] - ref).reshape(-1, cfg.head_dim).max(1)
        den = np.abs(ref).reshape(-1, cfg.head_dim).max(1)
        worst = max(worst, float((err / den).max()))
        layers += 1
    step_s = t_total / layers * L
    return {"cpu_baseline": {"value": prefill_flops(w) / step_s / 1e12, "unit": "TFLOP/s",
                             "cores": 1, "kind": "port", "us_per_token": step_s * 1e6 / n,
                             "sample": f"{layers} of {L} layers of the {n}-token prefill, oracle "
                                       f"on 1 thread, extrapolated"},
            "parity_normwise_max": worst}


def host_norms(dev, L, D):
    """Host copies of a QK-norm workload's [L][D] weights (None, None if none)."""
    if dev[0] is None:
        return None, None
    return (dev[0].download(np.float32, (L, D)), dev[1].download(np.float32, (L, D)))


def norm_args(w, qn, kn, layer):
    return {} if qn is None else dict(q_norm=qn[layer], k_norm=kn[layer], eps=w["qkn"])


def cpu_baseline(P, w, res, budget_s=12.0):
    """The oracle on one host thread over a bounded sample of the workload, and
    a parity spot check of the GPU output of the same step."""
    from oracle import oracle as O
    cfg, dkey, dval, (dq, dk, dv, dout), cos_t, sin_t, d_qn, d_kn = res.pop("_cpu_inputs")
    L, pos = cfg.n_layers, w["pos"]
    kc = dkey.download(np.uint16, (cfg.cache_elems,))
    vc = dval.download(np.uint16, (cfg.cache_elems,))
    q = dq.download(np.float32, (L, cfg.q_dim))
    k = dk.download(np.float32, (L, cfg.kv_dim))
    v = dv.download(np.float32, (L, cfg.kv_dim))
    gpu_out = dout.download(np.float32, (L, cfg.q_dim))
    shp = O.Shape(L, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
                  cfg.rope_freq_base, cfg.rope_type)
    qn, kn = host_norms((d_qn, d_kn), L, cfg.head_dim)
    tokens, t_total, worst = 0, 0.0, 0.0
    layers_done = 0
    while t_total < budget_s and tokens < 50:
        for l in range(L):
            qi, ki = q[l].copy(), k[l].copy()
            t0 = time.perf_counter()
            ref = O.attn_decode(shp, l, pos, qi, ki, v[l], kc, vc, cos_t, sin_t,
                                **norm_args(w, qn, kn, l))
            t_total += time.perf_counter() - t0
            layers_done += 1
            if tokens == 0:
                err = np.abs(gpu_out[l] - ref).reshape(-1, cfg.head_dim).max(1)
                den = np.abs(ref).reshape(-1, cfg.head_dim).max(1)
                worst = max(worst, float((err / den).max()))
            if t_total >= budget_s:
                break
        tokens += 1
    token_s = t_total / layers_done * L
    algo = decode_bytes(w)
    # head-parallel upper bound: the same per-head arithmetic over n host
    # threads (the reference runs its attention on one thread whatever -j)
    n_thr = min(os.cpu_count() or 1, HOST_THREADS_MAX)
    t_mt, mt_layers = 0.0, 0
    while qn is None and t_mt < budget_s / 2 and mt_layers < 4 * L:
        l = mt_layers % L
        qi, ki = q[l].copy(), k[l].copy()
        t0 = time.perf_counter()
        O.attn_decode_mt(shp, l, pos, qi, ki, v[l], kc, vc, cos_t, sin_t, n_thr)
        t_mt += time.perf_counter() - t0
        mt_layers += 1
    out = {
        "cpu_baseline": {"value": algo / token_s / 1e9, "unit": "GB/s", "cores": 1,
                         "kind": "port", "us_per_token": token_s * 1e6,
                         "sample": f"{layers_done} layer-steps ({layers_done / L:.2f} tokens) of "
                                   f"{w['L']}-layer decode at pos {pos}, oracle on 1 thread"},
        "host": host_info(),
        "parity_normwise_max": worst,
    }
    if mt_layers == 0:   # the head-parallel oracle has no QK-norm form
        return out
    token_mt = t_mt / mt_layers * L
    return {
        "cpu_baseline": {"value": algo / token_s / 1e9, "unit": "GB/s", "cores": 1,
                         "kind": "port", "us_per_token": token_s * 1e6,
                         "sample": f"{layers_done} layer-steps ({layers_done / L:.2f} tokens) of "
                                   f"{w['L']}-layer decode at pos {pos}, oracle on 1 thread"},
        "cpu_baseline_head_parallel": {
            "value": algo / token_mt / 1e9, "unit": "GB/s", "cores": n_thr, "kind": "port",
            "us_per_token": token_mt * 1e6,
            "sample": f"{mt_layers} layer-steps of the same decode, q heads split over "
                      f"{n_thr} threads: an upper bound, not the reference's own parallelism"},
        "host": host_info(),
        "parity_normwise_max": worst,
    }


def host_info():
    """nproc, CPU model and C library of the machine the CPU legs ran on."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        libc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        libc = None
    return {"nproc": os.cpu_count(), "cpu_model": model, "libc": libc}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="tinyllama_decode_pos2047",
                    choices=sorted(WORKLOADS) + [GEMV_WORKLOAD, FWD_WORKLOAD])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the secondary prefill measurement")
    ap.add_argument("--no-gemv", action="store_true",
                    help="skip the weight-GEMV measurement")
    ap.add_argument("--no-forward", action="store_true",
                    help="skip the whole-forward-pass measurement")
    ap.add_argument("--prompt", type=int, default=128,
                    help="prompt tokens of the forward-pass workload")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only: the attention block would shard by kv head "
                                   "(no exchange) or by sequence (one merge of the split "
                                   "partials per layer); neither is built",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import picolm_amd as P
    P.init(0)
    if args.workload == GEMV_WORKLOAD:   # the weight GEMVs of one token as the headline
        steps = max(1, args.steps // 50)
        gres = run_gemv(P, steps, min(args.warmup, 3))
        gextra = {} if args.no_cpu else cpu_baseline_gemv(gres)
        gres.pop("_inputs", None)
        line = {"metric": METRIC, "value": gres.pop("gbs"), "unit": "GB/s", "n_gpus": 1,
                "steps": steps, "warmup": min(args.warmup, 3),
                "ms_per_step": gres["us_per_token"] / 1e3, "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                "config": {"workload": GEMV_WORKLOAD, "matrices": len(gemv_matrices()),
                           **GEMV_TOKEN, "types": "Q4_K (q,k,o,gate,up), Q6_K (v,down,output)"}}
        line.update(gres)
        line.update(gextra)
        print(json.dumps(line), flush=True)
        return
    if args.workload == FWD_WORKLOAD:   # the whole forward pass as the headline
        n_decode = max(8, min(args.steps, 256))
        fres = run_forward(P, n_prompt=max(8, args.prompt), n_decode=n_decode)
        fextra = {} if args.no_cpu else cpu_baseline_forward(fres)
        fres.pop("_check", None)
        line = {"metric": METRIC, "value": fres.pop("decode_tok_s"), "unit": "tok/s",
                "n_gpus": 1, "steps": n_decode, "warmup": 4,
                "ms_per_step": fres["decode_us_per_token"] / 1e3, "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                "config": {"workload": FWD_WORKLOAD, **fres.pop("config")}}
        line.update(fres)
        line.update(fextra)
        print(json.dumps(line), flush=True)
        return
    w = WORKLOADS[args.workload]
    if "n" in w:   # a prefill workload as the headline
        res = run_prefill(P, w, max(1, args.steps // 10), args.warmup)
        extra = {} if args.no_cpu else cpu_baseline_prefill(P, w, res)
        res.pop("_copies", None)
        res.pop("_norms", None)
        line = {"metric": METRIC, "value": res.pop("tflops"), "unit": "TFLOP/s", "n_gpus": 1,
                "steps": max(1, args.steps // 10), "warmup": args.warmup,
                "ms_per_step": res["us_per_step"] / 1e3, "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic",
                "config": {"workload": args.workload, "n_layers": w["L"], "n_heads": w["Hq"],
                           "n_kv_heads": w["Hkv"], "head_dim": w["D"], "max_seq_len": w["S"],
                           "start_pos": w["start"], "n_tokens": w["n"],
                           "rope_theta": w["theta"], "rope_type": w.get("rt", 0),
                           "qk_norm_eps": w.get("qkn"), "batch": 1}}
        line.update(res)
        line.update(extra)
        print(json.dumps(line), flush=True)
        return
    res = run_decode(P, w, args.steps, args.warmup, args.workload)
    extra = {}
    if not args.no_cpu:
        extra = cpu_baseline(P, w, res)
    else:
        res.pop("_cpu_inputs", None)
    line = {
        "metric": METRIC,
        "value": res.pop("value"),
        "unit": res.pop("unit"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": args.workload, "n_layers": w["L"], "n_heads": w["Hq"],
                   "n_kv_heads": w["Hkv"], "head_dim": w["D"], "max_seq_len": w["S"],
                   "pos": w["pos"], "rope_theta": w["theta"], "rope_type": w.get("rt", 0),
                   "qk_norm_eps": w.get("qkn"), "batch": 1},
    }
    line["hbm_frac"] = res["roofline"]["frac"]
    line.update(res)
    line.update(extra)
    if not args.no_prefill:
        # the metric's prefill half: TinyLlama-shaped 512-token causal prefill
        pw = WORKLOADS["tinyllama_prefill_512"]
        pres = run_prefill(P, pw, 20, 3)
        pextra = {} if args.no_cpu else cpu_baseline_prefill(P, pw, pres, budget_s=4.0)
        pres.pop("_copies", None)
        pres.pop("_norms", None)
        pres["workload"] = "tinyllama_prefill_512"
        pres.update(pextra)
        line["prefill"] = pres
    if not args.no_gemv:
        # the gpu_try_matmul path: every weight GEMV of one TinyLlama token
        gres = run_gemv(P, 10, 2)
        gextra = {} if args.no_cpu else cpu_baseline_gemv(gres)
        gres.pop("_inputs", None)
        gres["workload"] = GEMV_WORKLOAD
        gres.update(gextra)
        line["gemv"] = gres
    if not args.no_forward:
        # the whole forward pass on the device (gpu_try_forward's path)
        fres = run_forward(P)
        h_fwd = fres["_check"][0]
        fextra = {} if args.no_cpu else cpu_baseline_forward(fres)
        if not args.no_cpu and "cpu_baseline" in line:
            # the headline's baseline from the reference itself where it runs
            refb = cpu_reference_attention(h_fwd, w)
            if refb is not None:
                line["cpu_baseline_port"] = line["cpu_baseline"]
                line["cpu_baseline"] = refb
        fres.pop("_check", None)
        fres.update(fextra)
        line["forward"] = fres
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
