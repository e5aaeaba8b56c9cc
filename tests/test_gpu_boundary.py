"""The gpu.h-style boundary (gpu_hip.c) on the GPU, driven from C by
tests/c/test_gpu_hip the way picolm's forward passes would call it.

Checks: every call handled (0), prefill and decode outputs against the
oracle, the host KV cache (kept authoritative by the boundary) bit-equal to
the oracle's, download/upload round trips for kvcache_save/load, Qwen3
layers (non-null attn_q_norm: QK-norm before RoPE with the layer's weights
and rms_norm_eps) mixed with plain ones, and the fallback switches:
PICOLM_HIP_DISABLE=1 (all -1, nothing touched) and PICOLM_GPU_LAYERS=1
(later layers -1, their rows untouched).
"""
import os
import subprocess

import numpy as np
import pytest

from attn_check import assert_attn_close
from conftest import ROOT

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "c", "test_gpu_hip")


EPS = 1e-6  # Qwen3's rms_norm_eps


def run_case(tmp_path, dims, theta, P, T, seed, env_extra=None, qkn_mask=0):
    L, Hq, Hkv, D, S, rt = dims
    rng = np.random.default_rng(seed)
    q_dim, kv_dim = Hq * D, Hkv * D
    pq = rng.standard_normal((L, P, q_dim), dtype=np.float32)
    pk = rng.standard_normal((L, P, kv_dim), dtype=np.float32)
    pv = rng.standard_normal((L, P, kv_dim), dtype=np.float32)
    dq = rng.standard_normal((T, L, q_dim), dtype=np.float32)
    dk = rng.standard_normal((T, L, kv_dim), dtype=np.float32)
    dv = rng.standard_normal((T, L, kv_dim), dtype=np.float32)
    qn = (1.0 + 0.5 * rng.standard_normal((L, D))).astype(np.float32)
    kn = (1.0 + 0.5 * rng.standard_normal((L, D))).astype(np.float32)
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        np.array([L, Hq, Hkv, D, S, rt, P, T, qkn_mask], np.int32).tofile(f)
        np.array([theta, EPS], np.float32).tofile(f)
        for a in (pq, pk, pv, dq, dk, dv, qn, kn):
            a.tofile(f)
    env = dict(os.environ)
    env.update(env_extra or {})
    print(f"[case] dims {dims} P {P} T {T} qkn {qkn_mask:#x} env {env_extra}", flush=True)
    r = subprocess.run([EXE, str(fin), str(fout)], env=env, capture_output=True, text=True,
                       timeout=240)
    assert r.returncode == 0, r.stderr
    buf = open(fout, "rb").read()
    off = 0

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(buf, dtype=dtype, count=count, offset=off)
        off += a.nbytes
        return a
    rc = take(np.int32, 4)
    rc_pre = take(np.int32, L)
    rc_dec = take(np.int32, T * L).reshape(T, L)
    out_pre = take(np.float32, L * P * q_dim).reshape(L, P, q_dim)
    out_dec = take(np.float32, T * L * q_dim).reshape(T, L, q_dim)
    n = L * S * kv_dim
    kc = take(np.uint16, n)
    vc = take(np.uint16, n)
    return (rc, rc_pre, rc_dec, out_pre, out_dec, kc, vc), (pq, pk, pv, dq, dk, dv, qn, kn)


def oracle_run(O, dims, theta, inputs, layers_gpu, qkn_mask=0):
    """Reference semantics for the layers that ran on the GPU; layers that fell
    back are left untouched (the harness skips the CPU block)."""
    L, Hq, Hkv, D, S, rt = dims
    pq, pk, pv, dq, dk, dv, qn, kn = inputs

    def norms(l):
        if (qkn_mask >> l) & 1:
            return dict(q_norm=qn[l], k_norm=kn[l], eps=EPS)
        return {}
    P, T = pq.shape[1], dq.shape[0]
    shp = O.Shape(L, Hq, Hkv, D, S, theta, rt)
    cos_t, sin_t = O.rope_tables(S, D, theta)
    kc = np.zeros(L * S * Hkv * D, np.uint16)
    vc = kc.copy()
    pre = np.zeros((L, P, Hq * D), np.float32)
    dec = np.zeros((T, L, Hq * D), np.float32)
    # the head-parallel form is bit-identical to attn_prefill; long prompts
    # need its threads to finish in seconds
    nthr = min(16, os.cpu_count() or 1)
    for l in layers_gpu:
        pre[l] = O.attn_prefill_mt(shp, l, 0, P, pq[l].copy(), pk[l].copy(), pv[l], kc, vc,
                                   cos_t, sin_t, nthr, **norms(l))
    for t in range(T):
        for l in layers_gpu:
            dec[t, l] = O.attn_decode(shp, l, P + t, dq[t, l].copy(), dk[t, l].copy(), dv[t, l],
                                      kc, vc, cos_t, sin_t, **norms(l))
    return pre, dec, kc, vc


CASES = [
    ((3, 32, 4, 64, 512, 0), 1e4, 200, 5),     # TinyLlama head layout
    ((2, 32, 8, 64, 600, 0), 5e5, 257, 3),     # Llama-3.2 head layout
    ((2, 32, 32, 128, 300, 0), 1e4, 90, 4),    # Llama-2 MHA
    ((2, 16, 2, 64, 128, 1), 1e6, 60, 3),      # QWEN rotation
    ((2, 8, 2, 96, 300, 0), 1e4, 90, 3),       # head_dim 96 (generic kernels)
    # 17 MB of out and rows back per prefill call: the DMA copies, not the copy kernel
    ((1, 32, 32, 128, 600, 0), 1e4, 520, 2),   # Llama-2 MHA, long prompt
]


@pytest.mark.parametrize("dims,theta,P,T", CASES)
def test_boundary_prefill_then_decode(tmp_path, oracle_mod, dims, theta, P, T):
    (rc, rc_pre, rc_dec, out_pre, out_dec, kc, vc), inputs = run_case(tmp_path, dims, theta, P,
                                                                        T, seed=P + T)
    L, D = dims[0], dims[3]
    assert list(rc) == [0, 0, 0, 0], rc
    assert np.all(rc_pre == 0) and np.all(rc_dec == 0)
    pre, dec, okc, ovc = oracle_run(oracle_mod, dims, theta, inputs, range(L))
    for l in range(L):
        assert_attn_close(out_pre[l], pre[l], D, 1e-3, f"prefill layer {l}")
        for t in range(T):
            assert_attn_close(out_dec[t, l], dec[t, l], D, 1e-3, f"decode t{t} layer {l}")
    assert np.array_equal(kc, okc) and np.array_equal(vc, ovc)


QKN_CASES = [
    ((3, 16, 8, 128, 400, 1), 1e6, 150, 4, 0b111),  # Qwen3-0.6B head layout, every layer
    ((3, 32, 4, 64, 300, 1), 1e6, 97, 3, 0b101),    # QK-norm layers mixed with plain ones
    ((2, 8, 4, 80, 200, 1), 1e6, 60, 3, 0b11),      # head_dim 80 (generic kernels)
]


@pytest.mark.parametrize("dims,theta,P,T,mask", QKN_CASES)
def test_boundary_qk_norm_layers(tmp_path, oracle_mod, dims, theta, P, T, mask):
    (rc, rc_pre, rc_dec, out_pre, out_dec, kc, vc), inputs = run_case(
        tmp_path, dims, theta, P, T, seed=P * T, qkn_mask=mask)
    L, D = dims[0], dims[3]
    assert list(rc) == [0, 0, 0, 0], rc
    assert np.all(rc_pre == 0) and np.all(rc_dec == 0)
    pre, dec, okc, ovc = oracle_run(oracle_mod, dims, theta, inputs, range(L), qkn_mask=mask)
    for l in range(L):
        assert_attn_close(out_pre[l], pre[l], D, 1e-3, f"prefill layer {l}")
        for t in range(T):
            assert_attn_close(out_dec[t, l], dec[t, l], D, 1e-3, f"decode t{t} layer {l}")
    assert np.array_equal(kc, okc) and np.array_equal(vc, ovc)


# Long contexts: the decode launch splits past 512 positions and its merge
# writes out into the pinned staging; TinyLlama heads at S 2048, a prompt
# of P tokens through the prefill hook, then T decode steps from position P.
LONG_CASES = [
    ((2, 32, 4, 64, 2048, 0), 1e4, 700, 2),    # decode at 700 and 701
    ((2, 32, 4, 64, 2048, 0), 1e4, 2047, 1),   # decode at 2047, the last cache row
]


@pytest.mark.parametrize("dims,theta,P,T", LONG_CASES, ids=["pos700", "pos2047"])
def test_boundary_long_context_decode(tmp_path, oracle_mod, dims, theta, P, T):
    test_boundary_prefill_then_decode(tmp_path, oracle_mod, dims, theta, P, T)


def test_boundary_disabled_falls_back_untouched(tmp_path, oracle_mod):
    dims, theta, P, T = CASES[0]
    (rc, rc_pre, rc_dec, out_pre, out_dec, kc, vc), _ = run_case(
        tmp_path, dims, theta, 40, 2, seed=1, env_extra={"PICOLM_HIP_DISABLE": "1"})
    assert rc[0] == -1 and rc[1] == -1 and rc[2] == -1 and rc[3] == -1
    assert np.all(rc_pre == -1) and np.all(rc_dec == -1)
    assert not out_pre.any() and not out_dec.any()
    assert not kc.any() and not vc.any()


def test_boundary_gpu_layers_limit(tmp_path, oracle_mod):
    dims, theta, P, T = CASES[0]
    L, D = dims[0], dims[3]
    (rc, rc_pre, rc_dec, out_pre, out_dec, kc, vc), inputs = run_case(
        tmp_path, dims, theta, 70, 3, seed=2, env_extra={"PICOLM_GPU_LAYERS": "1"})
    assert list(rc) == [0, 0, 0, 0], rc     # download / upload round trips hold
    assert rc_pre[0] == 0 and np.all(rc_pre[1:] == -1)
    assert np.all(rc_dec[:, 0] == 0) and np.all(rc_dec[:, 1:] == -1)
    pre, dec, okc, ovc = oracle_run(oracle_mod, dims, theta, inputs, [0])
    assert_attn_close(out_pre[0], pre[0], D, 1e-3, "prefill layer 0")
    for t in range(3):
        assert_attn_close(out_dec[t, 0], dec[t, 0], D, 1e-3, f"decode t{t} layer 0")
    assert not out_pre[1:].any() and not out_dec[:, 1:].any()
    # the CPU layers' rows (the harness's stand-in pattern) survive
    # gpu_kv_download: only the device's layers are copied back
    S, kv_dim, n_pos = dims[4], dims[2] * D, 73
    ok, ov = okc.reshape(L, S, kv_dim), ovc.reshape(L, S, kv_dim)
    r = np.arange(n_pos)[:, None]
    i = np.arange(kv_dim)[None, :]
    for l in range(1, L):
        ok[l, :n_pos] = 0x3C00 | ((l + 3 * r + i) & 0xFF)
        ov[l, :n_pos] = 0x4000 | ((l + 5 * r + i) & 0xFF)
    assert np.array_equal(kc, okc) and np.array_equal(vc, ovc)
