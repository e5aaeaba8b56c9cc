"""Benchmark of picolm's attention block on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]
                    [--tune KEY=VALUE ...]   (plh_set_tuning before the run, for sweeps)

Prints one JSON line.  The headline (the contract keys, `roofline`,
`cpu_baseline`) is TinyLlama-1.1B-shaped decode at position 2047 (22 layers,
32 q heads, 4 kv heads, head_dim 64, FP16 cache of 2048 rows): a step is one
token's decode attention over all 22 layers -- one plh_attn_decode call (one
stream-K launch at this shape, the split merge inside it) -- with inputs
resident in HBM.  The same line carries every
workload of the attention block's benchmark set, each measured the same way:

  cfg1  TinyLlama decode at pos 256            HBM-bound
  cfg2  TinyLlama decode at pos 2047           HBM-bound (the headline)
  cfg3  TinyLlama causal prefill of 512 tokens MFMA work, HBM roof at fp32 I/O
  cfg4  Llama-3.2-1B decode at pos 8191        HBM-bound
  cfg5a Llama-2-7B decode at pos 4095          HBM-bound
  cfg5b Llama-2-7B causal prefill of 1024      MFMA work, HBM roof at fp32 I/O

Method (device):
  * inputs rotated over enough copies (>= 512 MiB in all) that the 256 MiB
    Infinity Cache cannot serve a step from the previous one; K timed steps
    captured in one HIP graph, replayed untimed until SETTLE_S of device work
    has run, then once timed between device synchronisations (MFMA-heavy
    prefill runs up to 25% slower for the first ~30 ms after the GPU idles,
    a clock transient that settles whatever the kernel; the memory- and
    latency-bound decode, GEMV and forward steps show none);
    ms_per_step = wall clock / K, roofline.achieved =
    algorithmic bytes (decode) or causal-pair flops (prefill) / the mean step
    time from HIP events recorded on the library stream (the stream the
    kernels run on);
  * decode bytes per token, all layers: L * [(pos+1)*2*Hkv*D*2 (K+V rows read)
    + Hq*D*4 + 2*Hkv*D*4 (q, k, v in) + 2*Hkv*D*2 (row written) + Hq*D*4
    (out)]; prefill flops: L * Hq * 4D * sum_{i<N}(start+i+1) (causal pairs);
    prefill roof: the HBM roof at its arithmetic intensity (fp32 q/k/v/out),
    with the fraction of the fp16 MFMA peak beside it;
  * per_layer: the same token (prompt) as L one-layer calls, how a per-layer
    forward pass issues them, graph-replayed;
  * traffic: HBM bytes per launch of the dominant kernel from rocprofv3 --pmc
    (FETCH_SIZE, WRITE_SIZE, calibrated on a copy kernel), read from
    profiles/<workload>_traffic.json, null when none was measured;
  * boundary: the gpu.h-style hooks end to end (tests/c/bench_boundary: host
    q/k/v in, host output and cache rows back over PCIe) -- the latency
    picolm's own call sites would see; never the headline value; with it
    matmul_hook, gpu_try_matmul for every projection of one TinyLlama token
    (tests/c/bench_matmul), and forward_hook, gpu_try_forward,
    gpu_try_forward_prefill, gpu_kv_download and gpu_kv_upload of a
    TinyLlama-shaped model (tests/c/bench_forward).
Method (CPU baseline, kind "reference"): picolm's own attention code, i.e.
its model_forward_ex / model_forward_prefill compiled from its sources into
oracle/_ref, on the host, median of 5 runs after 1 warm-up, over a bounded
sample that the `sample` field names:
  * decode: a 2-layer model of the workload's attention shape with rows
    0..pos-1 of N(0,1) fp16, the forward at position pos minus the same
    forward at position 0 (the attention loop is the only part whose cost
    depends on pos), scaled to L layers; the attention loop runs on one
    thread whatever picolm's -j (model.c:848-892);
  * prefill: model_forward_prefill (projections at a small width included)
    of a 1-layer model with a slice of the workload's q heads (same head_dim,
    same GQA group), scaled to all heads and layers.
Beside it, cpu_baseline.head_parallel_upper_bound (kind "port"): the oracle's
restatement of the same attention with the q heads split over the host's
threads (bit-identical output), an upper bound for a parallel CPU attention
and not the reference's own parallelism (decode: 2 layers at pos; prefill:
one layer of the prompt; both scaled to all layers).
The oracle (the restatement in C, test infrastructure) checks the GPU outputs
of a sample layer (parity_normwise_max).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "attn µs/token + KV GB/s (% HBM peak) decode; prefill TFLOP/s (% MFMA)"
HBM_PEAK_GBS = 8000.0
MALL_DEFEAT_BYTES = 512 << 20
# untimed replays before each timed one, in seconds of device work
SETTLE_S = 0.1
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
# the benchmark set, in the order of the configs it is quoted on
CFG_SET = [("cfg1", "tinyllama_decode_pos256"), ("cfg2", "tinyllama_decode_pos2047"),
           ("cfg3", "tinyllama_prefill_512"), ("cfg4", "llama32_decode_pos8191"),
           ("cfg5a", "llama2_decode_pos4095"), ("cfg5b", "llama2_prefill_1024")]
HEADLINE = "tinyllama_decode_pos2047"
# CPU-baseline samples: decode layers; prefill (q heads, kv heads) of a 1-layer model
CPU_DECODE_LAYERS = 2
CPU_PREFILL_HEADS = {"tinyllama_prefill_512": (8, 1), "llama2_prefill_1024": (4, 4),
                     "qwen3_prefill_512": (2, 1)}


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


def run_gemv(P, steps, warmup, exact=False, inputs=None):
    """One step = every weight GEMV of one token (155 launches, device
    pointers, graph-replayed); the 670 MB of weights exceed the Infinity
    Cache, so each step streams them from HBM.  exact: the reference's AVX2
    summation order (plh_set_tuning key 10) instead of the default fast one;
    inputs: the matrices and vectors of an earlier call, reused."""
    P.check(P.lib.plh_set_tuning(10, 1 if exact else 0), "plh_set_tuning")
    try:
        return _run_gemv(P, steps, warmup, inputs)
    finally:
        P.check(P.lib.plh_set_tuning(10, 0), "plh_set_tuning")


def _run_gemv(P, steps, warmup, inputs):
    from picolm_amd import gemv as G
    from picolm_amd import synth as S
    if inputs is not None:
        return _time_gemv(P, steps, warmup, *inputs)
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
    return _time_gemv(P, steps, warmup, mats, host, dev, xs, outs)


def _time_gemv(P, steps, warmup, mats, host, dev, xs, outs):
    from picolm_amd import gemv as G

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
        "_inputs": (mats, host, dev, xs, outs),
    }


def cpu_baseline_gemv(res, budget_s=8.0):
    """The oracle's matmul (bit-identical to the reference's x86-64 AVX2
    vec_dot) on the host's cores, rows split over threads like the
    reference's matmul pool, over a bounded sample of the token's GEMVs;
    with the GPU outputs of the sampled GEMVs checked against it (normwise
    for the fast order, bit for bit for the exact one).  Returns the line's
    fields and the sampled references."""
    from oracle import oracle as O
    mats, host, dev, xs, outs = res["_inputs"]
    n_thr = min(os.cpu_count() or 1, HOST_THREADS_MAX)
    t_total, done_bytes, checked, exact, worst = 0.0, 0, 0, True, 0.0
    refs = []
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
        worst = max(worst, float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30)))
        refs.append((i, ref))
        checked += 1
    return {"cpu_baseline": {"value": done_bytes / t_total / 1e9, "unit": "GB/s",
                             "cores": n_thr, "kind": "port",
                             "us_per_token": t_total / done_bytes * gemv_bytes(mats) * 1e6,
                             "sample": f"the first {checked} of {len(mats)} GEMVs of the token, "
                                       f"oracle rows split over {n_thr} threads"},
            "parity_normwise_max_sampled": worst, "parity_bit_exact_sampled": exact,
            "parity_gemvs_checked": checked}, refs


def gemv_exact_order(P, gres, refs):
    """The same token's GEMVs in the exact order: timing and a bit-for-bit
    check of the sampled outputs against the oracle's."""
    mats, host, dev, xs, outs = gres["_inputs"]
    ex = run_gemv(P, 10, 2, exact=True, inputs=(mats, host, dev, xs, outs))
    ok = all(np.array_equal(outs[i].download(np.float32, (mats[i][2],)).view(np.uint32),
                            ref.view(np.uint32)) for i, ref in refs)
    return {"us_per_token": ex["us_per_token"], "gbs": ex["gbs"],
            "roofline_frac": ex["roofline"]["frac"], "parity_bit_exact_sampled": ok}


# The whole forward pass (model_forward on the device, plh_forward): a
# TinyLlama-1.1B-shaped Q4_K_M-style synthetic model (Q4_K embedding, q, k,
# o, gate, up; Q6_K v, down, output).
FWD_MODEL = dict(n_layers=22, n_embd=2048, n_ffn=5632, n_heads=32, n_kv_heads=4, head_dim=64,
                 vocab_size=32000, max_seq_len=2048)
FWD_WORKLOAD = "tinyllama_q4km_forward"
# plh_set_tuning settings from --tune (key -> value), reported in the line
TUNING = {}


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
    # the same tokens with the attention launches' L2 weight prefetch off
    # (tuning key 15), for comparison
    P.check(P.lib.plh_set_tuning(15, -1), "plh_set_tuning")
    try:
        for i in range(4):
            dm.forward(int(toks[i]), n_prompt + i)
        P.synchronize()
        e0.record()
        for i in range(n_decode):
            dm.forward(int(toks[4 + i]), n_prompt + 4 + i)
        e1.record()
        P.synchronize()
        dev_nopf_ms = e0.elapsed_ms(e1) / n_decode
    finally:
        P.check(P.lib.plh_set_tuning(15, TUNING.get(15, 0)), "plh_set_tuning")
    pos = n_prompt + 4 + n_decode
    tok = int(toks[-1])
    t0 = time.perf_counter()
    for i in range(n_decode):
        dm.forward(tok, pos + i)
        tok = int(np.argmax(dm.fetch_logits()))
    gen = (time.perf_counter() - t0) / n_decode
    # decode at the last cache row: rows 0..2046 of every layer hold N(0,1)
    # rounded to fp16 (what kvcache_load of a full context brings in), then
    # n_decode steps at position 2047, each attending over 2048 rows
    last = h.max_seq_len - 1
    kv = h.n_kv_heads * h.head_dim
    kfill = np.zeros((h.n_layers, h.max_seq_len, kv), np.float16)
    kfill[:, :last] = rng.standard_normal((h.n_layers, last, kv), dtype=np.float32)
    vfill = np.zeros_like(kfill)
    vfill[:, :last] = rng.standard_normal((h.n_layers, last, kv), dtype=np.float32)
    dm.load_cache(kfill.view(np.uint16).reshape(-1), vfill.view(np.uint16).reshape(-1))
    del kfill, vfill
    for i in range(4):
        dm.forward(int(toks[i]), last)
    P.synchronize()
    e0.record()
    for i in range(n_decode):
        dm.forward(int(toks[4 + i]), last)
    e1.record()
    P.synchronize()
    dev_last_ms = e0.elapsed_ms(e1) / n_decode
    # the same decode at position 2047 with the GEMVs in the exact order
    P.check(P.lib.plh_set_tuning(10, 1), "plh_set_tuning")
    try:
        dm.forward(int(toks[0]), last)
        P.synchronize()
        e0.record()
        for i in range(n_decode):
            dm.forward(int(toks[4 + i]), last)
        e1.record()
        P.synchronize()
        dev_last_exact_ms = e0.elapsed_ms(e1) / n_decode
    finally:
        P.check(P.lib.plh_set_tuning(10, 0), "plh_set_tuning")
    wb = h.weight_bytes_per_token()
    gbs = wb / (dev_ms * 1e-3) / 1e9
    res = {
        "workload": FWD_WORKLOAD,
        "config": dict(FWD_MODEL, types="Q4_K embd/q/k/o/gate/up, Q6_K v/down/output",
                       prompt=n_prompt),
        "decode_tok_s": 1.0 / wall,
        "decode_us_per_token": wall * 1e6,
        "decode_device_us_per_token": dev_ms * 1e3,
        "decode_device_us_per_token_no_l2_prefetch": dev_nopf_ms * 1e3,
        "decode_positions": [n_prompt + 4, n_prompt + 3 + n_decode],
        "decode_device_us_per_token_pos2047": dev_last_ms * 1e3,
        "decode_device_us_per_token_pos2047_exact_gemv": dev_last_exact_ms * 1e3,
        "gemv_order": "fast (int8 digits of x, integer dot products); prompt GEMVs exact",
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
    """(bytes, commit): HBM bytes per launch of the workload's dominant
    kernel, measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, calibrated
    on a copy kernel) and summarised in profiles/<name>_traffic.json, and the
    commit of the tree those counters were read on; (None, None) if not
    measured."""
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        return t.get("traffic_bytes"), t.get("commit")
    except (OSError, ValueError):
        return None, None


def norm_weights(P, w, rng):
    """Device [L][D] q and k norm weights for a QK-norm workload, else None."""
    if not w.get("qkn"):
        return None, None
    shape = (w["L"], w["D"])
    qn = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
    kn = (1.0 + 0.1 * rng.standard_normal(shape)).astype(np.float32)
    return P.DeviceBuffer.from_numpy(qn), P.DeviceBuffer.from_numpy(kn)


def timed_graph(P, launch, steps):
    """Captures `steps` calls of launch(i) in one graph, replays it untimed
    until SETTLE_S seconds have passed (at least once), then once timed;
    returns (wall seconds, event milliseconds) per step."""
    with P.Graph() as g:
        for i in range(steps):
            launch(i)
    t_end = time.perf_counter() + SETTLE_S
    while True:
        g.launch()
        P.synchronize()
        if time.perf_counter() >= t_end:
            break
    e0, e1 = P.Event(), P.Event()
    t0 = time.perf_counter()
    e0.record()
    g.launch()
    e1.record()
    P.synchronize()
    wall = (time.perf_counter() - t0) / steps
    return wall, e0.elapsed_ms(e1) / steps


def run_decode(P, w, steps, warmup, name, warm=False):
    """Decode workload on the device; returns the result dict and what the
    CPU legs need."""
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
    staging = P.DeviceBuffer(S * kv * 4)
    keys, vals = [], []
    for which in range(2):
        buf = P.DeviceBuffer(cache_bytes)
        buf.zero()
        for layer in range(L):   # one layer at a time keeps host memory small
            host = np.zeros((S, kv), np.float32)
            host[:pos] = rng.standard_normal((pos, kv), dtype=np.float32)
            staging.upload(host)
            P.f32_to_f16(staging.ptr, buf.ptr + layer * S * kv * 2, S * kv)
        (keys if which == 0 else vals).append(buf)
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

    for i in range(max(1, warmup)):   # also sizes the split workspace
        launch(i)
    P.synchronize()
    wall, k_ms = timed_graph(P, launch, steps)

    # the same token as L sequential one-layer calls (how a per-layer forward
    # pass calls the block)
    def launch_per_layer(i):
        c = i % n_copies
        q, k, v, o = qkv[c]
        for l in range(L):
            call(l, 1, q.ptr + l * cfg.q_dim * 4, k.ptr + l * kv * 4, v.ptr + l * kv * 4, c,
                 o.ptr + l * cfg.q_dim * 4)
    launch_per_layer(0)
    P.synchronize()
    _, pl_ms = timed_graph(P, launch_per_layer, max(1, min(steps, 20)))

    algo = decode_bytes(w)
    achieved = algo / (k_ms * 1e-3) / 1e9
    traffic = traffic_from_profiles(name)
    res = {
        "value": algo / wall / 1e9,
        "unit": "GB/s",
        "ms_per_step": wall * 1e3,
        "us_per_token": wall * 1e6,
        "kernel_us_mean": k_ms * 1e3,
        "algorithmic_bytes_per_step": algo,
        "cache_copies_rotated": n_copies,
        "gbs_wall": algo / wall / 1e9,
        "gbs_events": achieved,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "achieved_clock": "HIP events on the library stream",
                     "traffic": traffic[0], "traffic_commit": traffic[1]},
        "per_layer": {"us_per_token": pl_ms * 1e3, "gbs": algo / (pl_ms * 1e-3) / 1e9,
                      "launches_per_token": L},
    }
    if warm:
        # every step reuses copy 0: served from the Infinity Cache when it fits
        # in 256 MiB (reported apart, never the headline)
        def launch_warm(i):
            q, k, v, o = qkv[0]
            call(0, L, q.ptr, k.ptr, v.ptr, 0, o.ptr)
        _, warm_ms = timed_graph(P, launch_warm, steps)
        res["warm"] = {"us_per_token": warm_ms * 1e3, "gbs": algo / (warm_ms * 1e-3) / 1e9,
                       "note": "one cache copy reused every step: Infinity-Cache resident when "
                               "it fits in 256 MiB; not the headline"}
    res["_cpu_inputs"] = (cfg, keys[0], vals[0], qkv[0], d_qn, d_kn)
    return res


def run_prefill(P, w, steps, warmup, name):
    """One step = prefill of n prompt tokens over all layers (append kernel +
    causal attention kernel), inputs rotated over enough copies to defeat the
    Infinity Cache; the per-layer form as L one-layer calls."""
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

    def launch_per_layer(i):
        cache, q, k, v, o = copies[i % n_copies]
        for l in range(L):
            ln = {} if d_qn is None else dict(q_norm=d_qn.ptr + l * cfg.head_dim * 4,
                                              k_norm=d_kn.ptr + l * cfg.head_dim * 4,
                                              norm_eps=w["qkn"])
            P.prefill(cache, l, st, n, q.ptr + l * n * cfg.q_dim * 4,
                      k.ptr + l * n * cfg.kv_dim * 4, v.ptr + l * n * cfg.kv_dim * 4,
                      o.ptr + l * n * cfg.q_dim * 4, None, 1, **ln)

    for i in range(max(1, warmup)):
        launch(i)
    P.synchronize()
    wall, ms = timed_graph(P, launch, steps)
    launch_per_layer(0)
    P.synchronize()
    _, pl_ms = timed_graph(P, launch_per_layer, max(1, min(steps, 5)))
    flops = prefill_flops(w)
    algo_bytes = prefill_bytes(w)
    tfs = flops / (ms * 1e-3) / 1e12
    # the binding roof at this arithmetic intensity: HBM (expressed in TFLOP/s)
    # below the fp16 ridge, else the MFMA peak; MFMA utilisation beside it
    hbm_roof = flops / algo_bytes * HBM_PEAK_GBS / 1e3
    roof = min(MFMA_F16_PEAK_TFS, hbm_roof)
    traffic = traffic_from_profiles(name)
    return {
        "us_per_step": wall * 1e6,
        "us_per_token": wall * 1e6 / n,
        "tflops": tfs,
        "tflops_wall": flops / wall / 1e12,
        "tflops_events": tfs,
        "kernel_us_mean": ms * 1e3,
        "roofline": {"bound": "hbm" if hbm_roof < MFMA_F16_PEAK_TFS else "mfma",
                     "achieved": tfs, "peak": roof, "unit": "TFLOP/s", "frac": tfs / roof,
                     "achieved_clock": "HIP events on the library stream",
                     "traffic": traffic[0], "traffic_commit": traffic[1],
                     "achieved_gbs": algo_bytes / (ms * 1e-3) / 1e9,
                     "mfma_peak": MFMA_F16_PEAK_TFS, "mfma_frac": tfs / MFMA_F16_PEAK_TFS},
        "per_layer": {"us_per_step": pl_ms * 1e3, "tflops": flops / (pl_ms * 1e-3) / 1e12,
                      "launches_per_step": L},
        "algorithmic_flops_per_step": flops,
        "algorithmic_bytes_per_step": algo_bytes,
        "copies_rotated": n_copies,
        "_copies": copies,
        "_norms": (d_qn, d_kn),
    }


def n_host_threads():
    return min(os.cpu_count() or 1, HOST_THREADS_MAX)


def cpu_reference_decode(w, reps=5):
    """picolm's own decode attention (model.c:828-892) timed inside its
    model_forward_ex (oracle/_ref) on a CPU_DECODE_LAYERS-layer model of the
    workload's attention shape: the forward at position pos over rows
    0..pos-1 of N(0,1) fp16, minus the same forward at position 0, median of
    `reps` after one warm-up each, scaled to all layers."""
    from oracle import oracle as O
    if not O.ref_available():
        return None
    Ls, pos = CPU_DECODE_LAYERS, w["pos"]
    shp = O.Shape(Ls, w["Hq"], w["Hkv"], w["D"], w["S"], w["theta"], w.get("rt", 0))
    R = O.ref()
    R.ref_set_threads(1)   # the attention loop is single-threaded; idle pool threads would
    m = O.RefModel(shp, 0, seed=7)   # only compete with it
    try:
        rng = np.random.default_rng(4095)
        kv = w["Hkv"] * w["D"]
        for cache in (m.kc, m.vc):
            view = cache.reshape(Ls, w["S"], kv)
            for layer in range(Ls):
                view[layer, :pos] = O.f32_to_f16(
                    rng.standard_normal((pos, kv), dtype=np.float32)).reshape(pos, kv)
        for layer in range(Ls):
            q = rng.standard_normal(w["Hq"] * w["D"], dtype=np.float32)
            k = rng.standard_normal(kv, dtype=np.float32)
            v = rng.standard_normal(kv, dtype=np.float32)
            R.ref_set_decode_qkv(m.h, layer, q, k, v)
        out = np.empty(w["Hq"] * w["D"], np.float32)
        t_long, t_short = [], []
        for r in range(reps + 1):
            t0 = time.perf_counter()
            R.ref_decode(m.h, pos, Ls, out)
            t1 = time.perf_counter()
            R.ref_decode(m.h, 0, Ls, out)
            t2 = time.perf_counter()
            if r > 0:
                t_long.append(t1 - t0)
                t_short.append(t2 - t1)
    finally:
        R.ref_set_threads(1)
        m.close()
    attn_s = (float(np.median(t_long)) - float(np.median(t_short))) * w["L"] / Ls
    return {"value": decode_bytes(w) / attn_s / 1e9, "unit": "GB/s", "cores": 1,
            "kind": "reference", "us_per_token": attn_s * 1e6,
            "sample_layers": Ls, "total_layers": w["L"], "scale": w["L"] / Ls,
            "sample": f"model_forward_ex of a {Ls}-layer model of this attention shape at pos "
                      f"{pos} minus pos 0, median of {reps} after a warm-up, x{w['L'] // Ls} "
                      f"layers; 1 thread (picolm's pool runs matmul rows only, its attention "
                      f"loop is serial at any -j)"}


def cpu_reference_prefill(name, w, reps=5):
    """picolm's own model_forward_prefill (oracle/_ref) on a 1-layer model with
    a slice of the workload's q heads (same head_dim and GQA group; its
    projections at that small width included), median of `reps` after one
    warm-up, scaled to all heads and layers."""
    from oracle import oracle as O
    if not O.ref_available():
        return None
    hq, hkv = CPU_PREFILL_HEADS[name]
    n, st = w["n"], w["start"]
    shp = O.Shape(1, hq, hkv, w["D"], st + n, w["theta"], w.get("rt", 0))
    R = O.ref()
    R.ref_set_threads(1)
    m = O.RefModel(shp, 1, seed=9, w_scale=0.05)
    try:
        toks = (np.arange(n) * 7919 % (hq * w["D"])).astype(np.int32)
        logits = np.empty(hq * w["D"], np.float32)
        ts = []
        for r in range(reps + 1):
            t0 = time.perf_counter()
            R.ref_prefill(m.h, toks, n, st, logits)
            if r > 0:
                ts.append(time.perf_counter() - t0)
    finally:
        R.ref_set_threads(1)
        m.close()
    scale = (w["Hq"] / hq) * w["L"]
    step_s = float(np.median(ts)) * scale
    return {"value": prefill_flops(w) / step_s / 1e12, "unit": "TFLOP/s", "cores": 1,
            "kind": "reference", "us_per_token": step_s * 1e6 / n,
            "sample_layers": 1, "total_layers": w["L"], "sample_q_heads": hq,
            "total_q_heads": w["Hq"], "scale": scale,
            "sample": f"model_forward_prefill of a 1-layer model with {hq} q / {hkv} kv heads of "
                      f"head_dim {w['D']} ({n} tokens, projections included), median of {reps} "
                      f"after a warm-up, x{w['Hq'] // hq} heads x{w['L']} layers; 1 thread "
                      f"(picolm's pool runs matmul rows only, its attention loop is serial at "
                      f"any -j)"}


def cpu_head_parallel_decode(w, reps=7, warm=3):
    """Upper bound for a parallel CPU attention, not the reference's own
    parallelism (picolm's -j pool runs matmul rows only): the oracle's
    restatement of its decode attention (model.c:828-892) with the q heads
    split over the host's threads (orc_attn_decode_mt, bit-identical to the
    serial loop), CPU_DECODE_LAYERS layers at pos, median of `reps` after
    at least `warm` warm-up calls and 0.3 s of them, scaled to all layers
    (QK-norm, O(D) per head, left out)."""
    from oracle import oracle as O
    Ls, pos, S, D = CPU_DECODE_LAYERS, w["pos"], w["S"], w["D"]
    shp = O.Shape(Ls, w["Hq"], w["Hkv"], D, S, w["theta"], w.get("rt", 0))
    n_thr = n_host_threads()
    rng = np.random.default_rng(4096)
    kv = w["Hkv"] * D
    kc = np.zeros(Ls * S * kv, np.uint16)
    vc = np.zeros(Ls * S * kv, np.uint16)
    for cache in (kc, vc):
        view = cache.reshape(Ls, S, kv)
        for layer in range(Ls):
            view[layer, :pos] = O.f32_to_f16(
                rng.standard_normal((pos, kv), dtype=np.float32)).reshape(pos, kv)
    cos_t, sin_t = O.rope_tables(S, D, w["theta"])
    q = rng.standard_normal((Ls, w["Hq"] * D), dtype=np.float32)
    k = rng.standard_normal((Ls, kv), dtype=np.float32)
    v = rng.standard_normal((Ls, kv), dtype=np.float32)
    def once():
        qs, ks = q.copy(), k.copy()
        t0 = time.perf_counter()
        for layer in range(Ls):
            O.attn_decode_mt(shp, layer, pos, qs[layer], ks[layer], v[layer], kc, vc, cos_t,
                             sin_t, n_thr)
        return time.perf_counter() - t0

    # warm-up: at least `warm` calls and 0.3 s (idle cores take tens of ms to
    # come up to speed under new threads)
    t_end = time.perf_counter() + 0.3
    for r in range(warm):
        once()
    while time.perf_counter() < t_end:
        once()
    ts = [once() for _ in range(reps)]
    step_s = float(np.median(ts)) * w["L"] / Ls
    return {"value": decode_bytes(w) / step_s / 1e9, "unit": "GB/s", "cores": n_thr,
            "kind": "port", "us_per_token": step_s * 1e6,
            "sample_layers": Ls, "total_layers": w["L"], "scale": w["L"] / Ls,
            "sample": f"oracle decode attention at pos {pos} with q heads split over {n_thr} "
                      f"threads, {Ls} layers, median of {reps} after >= 0.3 s of warm-up, "
                      f"x{w['L'] // Ls} layers; upper bound, not the reference's own "
                      f"parallelism"}


def cpu_head_parallel_prefill(w, reps=3):
    """Upper bound for a parallel CPU prefill attention, not the reference's
    own parallelism: the oracle's restatement of model.c:1019-1090 for one
    layer with the attention split by q head over the host's threads
    (orc_attn_prefill_mt, bit-identical to the serial loop), QK-norm
    included where the workload has it, median of `reps` after a warm-up,
    scaled to all layers."""
    from oracle import oracle as O
    n, st, D = w["n"], w["start"], w["D"]
    shp = O.Shape(1, w["Hq"], w["Hkv"], D, st + n, w["theta"], w.get("rt", 0))
    n_thr = n_host_threads()
    rng = np.random.default_rng(1025)
    kv = w["Hkv"] * D
    kc = np.zeros((st + n) * kv, np.uint16)
    vc = np.zeros((st + n) * kv, np.uint16)
    if st:
        kc[: st * kv] = O.f32_to_f16(rng.standard_normal(st * kv, dtype=np.float32))
        vc[: st * kv] = O.f32_to_f16(rng.standard_normal(st * kv, dtype=np.float32))
    cos_t, sin_t = O.rope_tables(st + n, D, w["theta"])
    q = rng.standard_normal((n, w["Hq"] * D), dtype=np.float32)
    k = rng.standard_normal((n, kv), dtype=np.float32)
    v = rng.standard_normal((n, kv), dtype=np.float32)
    qn = kn = None
    if w.get("qkn"):
        qn = (rng.standard_normal(D) * 0.5 + 1.0).astype(np.float32)
        kn = (rng.standard_normal(D) * 0.5 + 1.0).astype(np.float32)
    ts = []
    for r in range(reps + 1):
        qs, ks = q.copy(), k.copy()
        t0 = time.perf_counter()
        O.attn_prefill_mt(shp, 0, st, n, qs, ks, v, kc, vc, cos_t, sin_t, n_thr, q_norm=qn,
                          k_norm=kn, eps=w.get("qkn") or 0.0)
        if r > 0:
            ts.append(time.perf_counter() - t0)
    step_s = float(np.median(ts)) * w["L"]
    return {"value": prefill_flops(w) / step_s / 1e12, "unit": "TFLOP/s", "cores": n_thr,
            "kind": "port", "us_per_token": step_s * 1e6 / n,
            "sample_layers": 1, "total_layers": w["L"], "scale": float(w["L"]),
            "sample": f"oracle prefill attention of one layer ({n} tokens from {st}) with q heads "
                      f"split over {n_thr} threads, median of {reps} after a warm-up, "
                      f"x{w['L']} layers; upper bound, not the reference's own parallelism"}


def decode_parity(P, w, res, layers=(0,)):
    """Normwise error of the GPU output of sample layers against the oracle."""
    from oracle import oracle as O
    cfg, dkey, dval, (dq, dk, dv, dout), d_qn, d_kn = res.pop("_cpu_inputs")
    L, pos = cfg.n_layers, w["pos"]
    kc = dkey.download(np.uint16, (cfg.cache_elems,))
    vc = dval.download(np.uint16, (cfg.cache_elems,))
    q = dq.download(np.float32, (L, cfg.q_dim))
    k = dk.download(np.float32, (L, cfg.kv_dim))
    v = dv.download(np.float32, (L, cfg.kv_dim))
    gpu_out = dout.download(np.float32, (L, cfg.q_dim))
    shp = O.Shape(L, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
                  cfg.rope_freq_base, cfg.rope_type)
    cos_t, sin_t = O.rope_tables(cfg.max_seq_len, cfg.head_dim, cfg.rope_freq_base)
    qn = None if d_qn is None else d_qn.download(np.float32, (L, cfg.head_dim))
    kn = None if d_kn is None else d_kn.download(np.float32, (L, cfg.head_dim))
    worst = 0.0
    for l in layers:
        extra = {} if qn is None else dict(q_norm=qn[l], k_norm=kn[l], eps=w["qkn"])
        ref = O.attn_decode(shp, l, pos, q[l].copy(), k[l].copy(), v[l], kc, vc, cos_t, sin_t,
                            **extra)
        err = np.abs(gpu_out[l] - ref).reshape(-1, cfg.head_dim).max(1)
        den = np.abs(ref).reshape(-1, cfg.head_dim).max(1)
        worst = max(worst, float((err / den).max()))
    return worst


def prefill_parity(P, w, res, layers=(0,)):
    from oracle import oracle as O
    cache, dq, dk, dv, dout = res.pop("_copies")[0]
    d_qn, d_kn = res.pop("_norms")
    cfg = cache.cfg
    L, n, st = cfg.n_layers, w["n"], w["start"]
    kc, vc = cache.fetch()
    shp = O.Shape(L, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
                  cfg.rope_freq_base, cfg.rope_type)
    cos_t, sin_t = O.rope_tables(cfg.max_seq_len, cfg.head_dim, cfg.rope_freq_base)
    qn = None if d_qn is None else d_qn.download(np.float32, (L, cfg.head_dim))
    kn = None if d_kn is None else d_kn.download(np.float32, (L, cfg.head_dim))
    worst = 0.0
    for l in layers:
        q = dq.download(np.float32, (n, cfg.q_dim), offset=l * n * cfg.q_dim * 4)
        k = dk.download(np.float32, (n, cfg.kv_dim), offset=l * n * cfg.kv_dim * 4)
        v = dv.download(np.float32, (n, cfg.kv_dim), offset=l * n * cfg.kv_dim * 4)
        gpu_out = dout.download(np.float32, (n, cfg.q_dim), offset=l * n * cfg.q_dim * 4)
        extra = {} if qn is None else dict(q_norm=qn[l], k_norm=kn[l], eps=w["qkn"])
        ref = O.attn_prefill(shp, l, st, n, q.copy(), k.copy(), v, kc, vc, cos_t, sin_t,
                             **extra)
        err = np.abs(gpu_out - ref).reshape(-1, cfg.head_dim).max(1)
        den = np.abs(ref).reshape(-1, cfg.head_dim).max(1)
        worst = max(worst, float((err / den).max()))
    return worst


def boundary_latency(w, reps=20):
    """gpu_try_attention (decode) or gpu_try_attention_prefill end to end,
    PCIe copies included, from tests/c/bench_boundary; None if not built."""
    exe = os.path.join(ROOT, "tests", "c", "bench_boundary")
    if not os.path.exists(exe):
        return None
    pos, n = (w["pos"], 0) if "pos" in w else (w["start"], w["n"])
    args = [exe] + [str(x) for x in (w["L"], w["Hq"], w["Hkv"], w["D"], w["S"], w["theta"], pos,
                                     n, reps)]
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"error": r.stderr.strip()[-200:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


def matmul_hook_latency(reps=10):
    """gpu_try_matmul over one TinyLlama-shaped token's 155 projections (host
    x in, host out back), from tests/c/bench_matmul; None if not built."""
    exe = os.path.join(ROOT, "tests", "c", "bench_matmul")
    if not os.path.exists(exe):
        return None
    args = [exe] + [str(x) for x in (22, 2048, 5632, 32, 4, 32000, reps)]
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"error": r.stderr.strip()[-200:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


def forward_hook_latency(reps=10):
    """gpu_try_forward (a decode token at position 257) and
    gpu_try_forward_prefill (a 128-token prompt) of a TinyLlama-shaped
    Q4_K_M model, logits, x and cache rows back in host memory, then
    gpu_kv_download / gpu_kv_upload of every layer's rows up to kv_pos
    (kvcache_save / kvcache_load coherence), from tests/c/bench_forward;
    None if not built."""
    exe = os.path.join(ROOT, "tests", "c", "bench_forward")
    if not os.path.exists(exe):
        return None
    args = [exe] + [str(x) for x in (22, 2048, 5632, 32, 4, 32000, 2048, 256, reps, 128)]
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"error": r.stderr.strip()[-200:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


def measure(P, name, steps, warmup, cpu, warm=False):
    """One workload: device figures, CPU baseline, parity sample."""
    w = WORKLOADS[name]
    if "n" in w:
        res = run_prefill(P, w, steps, warmup, name)
        if cpu:
            res["cpu_baseline"] = cpu_reference_prefill(name, w)
            if res["cpu_baseline"] is not None:
                res["cpu_baseline"]["head_parallel_upper_bound"] = cpu_head_parallel_prefill(w)
        res["parity_normwise_max"] = prefill_parity(P, w, res) if w["n"] <= 512 else None
        res.pop("_copies", None)
        res.pop("_norms", None)
    else:
        res = run_decode(P, w, steps, warmup, name, warm=warm)
        if cpu:
            res["cpu_baseline"] = cpu_reference_decode(w)
            if res["cpu_baseline"] is not None:
                res["cpu_baseline"]["head_parallel_upper_bound"] = cpu_head_parallel_decode(w)
        res["parity_normwise_max"] = decode_parity(P, w, res)
        res.pop("_cpu_inputs", None)
    return res


def workload_config(name):
    w = WORKLOADS[name]
    c = {"workload": name, "n_layers": w["L"], "n_heads": w["Hq"], "n_kv_heads": w["Hkv"],
         "head_dim": w["D"], "max_seq_len": w["S"], "rope_theta": w["theta"],
         "rope_type": w.get("rt", 0), "qk_norm_eps": w.get("qkn"), "batch": 1}
    if "pos" in w:
        c["pos"] = w["pos"]
    else:
        c["start_pos"], c["n_tokens"] = w["start"], w["n"]
    return c


def compact(tag, name, res):
    """The flat summary of one workload (the end of the bench line)."""
    rf, cb, pl = res["roofline"], res.get("cpu_baseline") or {}, res["per_layer"]
    out = {"cfg": tag, "w": name}
    if "tflops" in res:
        out.update(us_step=round(res["us_per_step"], 1), us_tok=round(res["us_per_token"], 3),
                   tfs=round(res["tflops"], 1), mfma_frac=round(rf["mfma_frac"], 4),
                   pl_us_step=round(pl["us_per_step"], 1))
    else:
        out.update(us_tok=round(res["us_per_token"], 2), gbs=round(res["value"], 1),
                   pl_us_tok=round(pl["us_per_token"], 1))
    out.update(kern_us=round(res["kernel_us_mean"], 2), frac=round(rf["frac"], 4), peak=rf["peak"],
               traffic=None if rf["traffic"] is None else int(rf["traffic"]),
               traffic_commit=rf.get("traffic_commit"),
               cpu_us_tok=None if not cb else round(cb["us_per_token"], 1),
               cpu_kind=cb.get("kind"),
               cpu_mt_us_tok=None if not cb.get("head_parallel_upper_bound")
               else round(cb["head_parallel_upper_bound"]["us_per_token"], 1),
               cpu_mt_cores=(cb.get("head_parallel_upper_bound") or {}).get("cores"),
               parity=None if res.get("parity_normwise_max") is None
               else float(f"{res['parity_normwise_max']:.2e}"))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=None,
                    choices=sorted(WORKLOADS) + [GEMV_WORKLOAD, FWD_WORKLOAD],
                    help="measure this workload alone (no benchmark set)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the GEMV, forward-pass and boundary-latency sections")
    ap.add_argument("--prompt", type=int, default=128,
                    help="prompt tokens of the forward-pass workload")
    ap.add_argument("--tune", action="append", default=[], metavar="KEY=VALUE",
                    help="plh_set_tuning(KEY, VALUE) before the run (repeatable)")
    args = ap.parse_args()
    for t in args.tune:
        k, _, v = t.partition("=")
        TUNING[int(k)] = int(v)
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU only: the attention block would shard by kv head "
                                   "(no exchange) or by sequence (one merge of the split "
                                   "partials per layer); neither is built",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import picolm_amd as P
    P.init(0)
    for k, v in TUNING.items():
        P.check(P.lib.plh_set_tuning(k, v), f"plh_set_tuning({k}, {v})")
    cpu = not args.no_cpu
    if args.workload == GEMV_WORKLOAD:   # the weight GEMVs of one token as the headline
        steps = max(1, args.steps // 50)
        gres = run_gemv(P, steps, min(args.warmup, 3))
        gextra = cpu_baseline_gemv(gres)[0] if cpu else {}
        gres.pop("_inputs", None)
        line = {"metric": METRIC, "value": gres.pop("gbs"), "unit": "GB/s", "n_gpus": 1,
                "steps": steps, "warmup": min(args.warmup, 3),
                "ms_per_step": gres["us_per_token"] / 1e3, "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                "config": {"workload": GEMV_WORKLOAD, "matrices": len(gemv_matrices()),
                           **GEMV_TOKEN, "types": "Q4_K (q,k,o,gate,up), Q6_K (v,down,output)"}}
        line.update(gres)
        line.update(gextra)
        if TUNING:
            line["tuning"] = {str(k): v for k, v in TUNING.items()}
        print(json.dumps(line), flush=True)
        return
    if args.workload == FWD_WORKLOAD:   # the whole forward pass as the headline
        n_decode = max(8, min(args.steps, 256))
        fres = run_forward(P, n_prompt=max(8, args.prompt), n_decode=n_decode)
        fextra = cpu_baseline_forward(fres) if cpu else {}
        fres.pop("_check", None)
        line = {"metric": METRIC, "value": fres.pop("decode_tok_s"), "unit": "tok/s",
                "n_gpus": 1, "steps": n_decode, "warmup": 4,
                "ms_per_step": fres["decode_us_per_token"] / 1e3, "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                "config": {"workload": FWD_WORKLOAD, **fres.pop("config")}}
        line.update(fres)
        line.update(fextra)
        if TUNING:
            line["tuning"] = {str(k): v for k, v in TUNING.items()}
        print(json.dumps(line), flush=True)
        return

    head = args.workload or HEADLINE
    w = WORKLOADS[head]
    hres = measure(P, head, args.steps, args.warmup, cpu, warm=args.workload is None)
    is_prefill = "n" in w
    line = {
        "metric": METRIC,
        "value": hres["tflops"] if is_prefill else hres["value"],
        "unit": "TFLOP/s" if is_prefill else "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": (hres["us_per_step"] / 1e3) if is_prefill else hres["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": workload_config(head),
        "roofline": hres["roofline"],
        "cpu_baseline": hres.get("cpu_baseline"),
    }
    line["value_clock"] = ("HIP events on the library stream" if is_prefill
                           else "host wall clock around the graph replay")
    for key in ("gbs_wall", "gbs_events", "tflops_wall", "tflops_events",
                "us_per_token", "us_per_step", "kernel_us_mean", "algorithmic_bytes_per_step",
                "algorithmic_flops_per_step", "cache_copies_rotated", "copies_rotated",
                "per_layer", "warm", "parity_normwise_max"):
        if key in hres:
            line[key] = hres[key]
    if cpu:
        line["host"] = host_info()
    if args.workload is not None:   # one workload alone (profiling runs)
        if TUNING:
            line["tuning"] = {str(k): v for k, v in TUNING.items()}
        print(json.dumps(line), flush=True)
        return

    # the rest of the benchmark set, each measured the same way
    results = {HEADLINE: hres}
    for tag, name in CFG_SET:
        if name == HEADLINE:
            continue
        # their own step counts (each step is short; the headline keeps --steps)
        steps = 20 if "n" in WORKLOADS[name] else 200
        results[name] = measure(P, name, steps, 5, cpu)
    pres = results["tinyllama_prefill_512"]
    # the metric's prefill half, flat (cfg3)
    line["prefill"] = {"workload": "tinyllama_prefill_512",
                       "us_per_step": pres["us_per_step"], "us_per_token": pres["us_per_token"],
                       "tflops": pres["tflops"], "roofline_frac": pres["roofline"]["frac"],
                       "roofline_peak": pres["roofline"]["peak"],
                       "mfma_frac": pres["roofline"]["mfma_frac"],
                       "traffic": pres["roofline"]["traffic"],
                       "per_layer_us_per_step": pres["per_layer"]["us_per_step"],
                       "cpu_us_per_token": (pres.get("cpu_baseline") or {}).get("us_per_token"),
                       "cpu_kind": (pres.get("cpu_baseline") or {}).get("kind"),
                       "parity_normwise_max": pres.get("parity_normwise_max")}
    if not args.no_extras:
        # the gpu.h-style hooks end to end (PCIe included), cfg1 / cfg2 decode, cfg3 prefill
        line["boundary"] = {tag: boundary_latency(WORKLOADS[name])
                            for tag, name in (("cfg1", "tinyllama_decode_pos256"),
                                              ("cfg2", "tinyllama_decode_pos2047"),
                                              ("cfg3", "tinyllama_prefill_512"))}
        line["matmul_hook"] = matmul_hook_latency()
        line["forward_hook"] = forward_hook_latency()
        # the gpu_try_matmul path: every weight GEMV of one TinyLlama token
        gres = run_gemv(P, 10, 2)
        gextra, refs = cpu_baseline_gemv(gres) if cpu else ({}, [])
        gres["exact_order"] = gemv_exact_order(P, gres, refs)
        gres.pop("_inputs", None)
        gres["workload"] = GEMV_WORKLOAD
        gres["order"] = "fast (int8 digits of x, integer dot products)"
        gres.update(gextra)
        line["gemv"] = gres
        # the whole forward pass on the device (gpu_try_forward's path)
        fres = run_forward(P)
        fextra = cpu_baseline_forward(fres) if cpu else {}
        fres.pop("_check", None)
        fres.update(fextra)
        line["forward"] = fres
    # last, so that a tail of the line holds it: the benchmark set, flat
    line["workloads"] = [compact(tag, name, results[name]) for tag, name in CFG_SET]
    if TUNING:
        line["tuning"] = {str(k): v for k, v in TUNING.items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
