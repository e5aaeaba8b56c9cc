"""Qwen3 QK-norm (model.c:807-817 decode, 1029-1037 prefill) on the GPU
against the oracle (pinned bit-exact to the reference in
tests/test_oracle_qknorm.py): attention outputs within the tolerance of
tests/attn_check.py, caches bit for bit -- the k rows are normalised,
rotated and rounded on the device with the reference's summation order.
"""
import numpy as np
import pytest

from attn_check import assert_attn_close, filled_cache, normal_f32

pytestmark = pytest.mark.gpu

EPS = 1e-6
# (L, Hq, Hkv, D, S, theta, rope_type)
CONFIGS = [
    (2, 16, 8, 128, 1024, 1e6, 1),   # Qwen3-0.6B head layout (QWEN rotation)
    (2, 32, 4, 128, 1024, 1e6, 1),   # GQA 8, head_dim 128
    (3, 32, 4, 64, 1024, 1e4, 0),    # LLaMA rotation with QK-norm, head_dim 64
]


def _weights(rng, L, D):
    qw = (rng.standard_normal((L, D)) * 0.5 + 1.0).astype(np.float32)
    kw = (rng.standard_normal((L, D)) * 0.5 + 1.0).astype(np.float32)
    return qw, kw


@pytest.mark.parametrize("dims", CONFIGS)
@pytest.mark.parametrize("pos", [0, 1, 300, 900])
def test_decode_qknorm(gpu, oracle_mod, dims, pos):
    O = oracle_mod
    L, Hq, Hkv, D, S, theta, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    rng = np.random.default_rng(pos * 7 + D)
    print(f"[case] decode qknorm {dims} pos {pos}", flush=True)
    kc, vc = filled_cache(O, cfg, pos, rng)
    q = normal_f32(rng, (L, cfg.q_dim), 3.0)
    k = normal_f32(rng, (L, cfg.kv_dim), 3.0)
    v = normal_f32(rng, (L, cfg.kv_dim))
    qw, kw = _weights(rng, L, D)
    cache = gpu.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv, dqw, dkw = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v, qw, kw))
    dout = gpu.DeviceBuffer(L * cfg.q_dim * 4)
    gpu.decode(cache, 0, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, L, q_norm=dqw.ptr,
               k_norm=dkw.ptr, norm_eps=EPS)
    gpu.synchronize()
    out = dout.download(np.float32, (L, cfg.q_dim))
    gk, gv = cache.fetch()
    cache.free()
    shp = O.Shape(L, Hq, Hkv, D, S, theta, rt)
    cos_t, sin_t = O.rope_tables(S, D, theta)
    rk, rv = kc.copy(), vc.copy()
    for l in range(L):
        ref = O.attn_decode(shp, l, pos, q[l].copy(), k[l].copy(), v[l], rk, rv, cos_t, sin_t,
                            q_norm=qw[l], k_norm=kw[l], eps=EPS)
        assert_attn_close(out[l], ref, D, what=f"decode qknorm layer {l}")
    assert np.array_equal(gk, rk) and np.array_equal(gv, rv)


@pytest.mark.parametrize("dims", CONFIGS)
def test_prefill_qknorm_chunks_then_decode(gpu, oracle_mod, dims):
    """Two prefill chunks (the second attends over the first through the
    cache) and a decode step after them, all with QK-norm."""
    O = oracle_mod
    L, Hq, Hkv, D, S, theta, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    rng = np.random.default_rng(D + rt)
    qw, kw = _weights(rng, L, D)
    dqw, dkw = gpu.DeviceBuffer.from_numpy(qw), gpu.DeviceBuffer.from_numpy(kw)
    shp = O.Shape(L, Hq, Hkv, D, S, theta, rt)
    cos_t, sin_t = O.rope_tables(S, D, theta)
    cache = gpu.KVCache(cfg)
    kc = np.zeros(L * S * cfg.kv_dim, np.uint16)
    vc = kc.copy()
    cache.load(kc, vc)
    start = 0
    for n in (77, 130):
        print(f"[case] prefill qknorm {dims} start {start} n {n}", flush=True)
        q = normal_f32(rng, (L, n, cfg.q_dim), 3.0)
        k = normal_f32(rng, (L, n, cfg.kv_dim), 3.0)
        v = normal_f32(rng, (L, n, cfg.kv_dim))
        dq, dk, dv = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v))
        dout = gpu.DeviceBuffer(L * n * cfg.q_dim * 4)
        gpu.prefill(cache, 0, start, n, dq.ptr, dk.ptr, dv.ptr, dout.ptr, None, L,
                    q_norm=dqw.ptr, k_norm=dkw.ptr, norm_eps=EPS)
        gpu.synchronize()
        out = dout.download(np.float32, (L, n, cfg.q_dim))
        for l in range(L):
            ref = O.attn_prefill(shp, l, start, n, q[l].copy(), k[l].copy(), v[l], kc, vc,
                                 cos_t, sin_t, q_norm=qw[l], k_norm=kw[l], eps=EPS)
            assert_attn_close(out[l], ref, D, what=f"prefill qknorm start {start} layer {l}")
        start += n
    gk, gv = cache.fetch()
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)
    # one decode step on top of the prefilled cache
    q = normal_f32(rng, (L, cfg.q_dim), 3.0)
    k = normal_f32(rng, (L, cfg.kv_dim), 3.0)
    v = normal_f32(rng, (L, cfg.kv_dim))
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = gpu.DeviceBuffer(L * cfg.q_dim * 4)
    gpu.decode(cache, 0, start, dq.ptr, dk.ptr, dv.ptr, dout.ptr, L, q_norm=dqw.ptr,
               k_norm=dkw.ptr, norm_eps=EPS)
    gpu.synchronize()
    out = dout.download(np.float32, (L, cfg.q_dim))
    for l in range(L):
        ref = O.attn_decode(shp, l, start, q[l].copy(), k[l].copy(), v[l], kc, vc, cos_t, sin_t,
                            q_norm=qw[l], k_norm=kw[l], eps=EPS)
        assert_attn_close(out[l], ref, D, what=f"decode after prefill layer {l}")
    gk, gv = cache.fetch()
    cache.free()
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)


def test_qknorm_needs_both_weights(gpu):
    cfg = gpu.AttnConfig(1, 16, 8, 128, 64, 1e6, 1)
    cache = gpu.KVCache(cfg)
    buf = gpu.DeviceBuffer(1 << 16)
    lib = gpu.lib
    rc = lib.plh_attn_decode_qknorm(1, 16, 8, 128, 64, 1, 0, 1, 3, buf.ptr, buf.ptr, buf.ptr,
                                    cache.key.ptr, cache.val.ptr, cache.cos.ptr, cache.sin.ptr,
                                    buf.ptr, buf.ptr, None, 1e-6)
    assert rc == -1 and b"both" in lib.plh_last_error()
    rc = lib.plh_attn_prefill_qknorm(1, 16, 8, 128, 64, 1, 0, 1, 0, 4, buf.ptr, buf.ptr,
                                     buf.ptr, cache.key.ptr, cache.val.ptr, cache.cos.ptr,
                                     cache.sin.ptr, buf.ptr, 16 * 128, None, buf.ptr, 1e-6)
    assert rc == -1 and b"both" in lib.plh_last_error()
    cache.free()


@pytest.mark.parametrize("tuning", [(5, 4), (6, 2), (6, 3)], ids=["chunks4", "ksplit2", "ksplit3"])
@pytest.mark.parametrize("dims", CONFIGS[:2])
def test_prefill_qknorm_one_layer_split(gpu, oracle_mod, dims, tuning):
    """One layer of a prompt whose heavy q blocks are split into 4-tile chunks
    (plh_set_tuning key 5) and merged, or run by K-split workgroups (key 6):
    QK-norm inside every chunk's or wave group's prologue."""
    O = oracle_mod
    L, Hq, Hkv, D, S, theta, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    rng = np.random.default_rng(D + 17)
    qw, kw = _weights(rng, L, D)
    dqw = gpu.DeviceBuffer.from_numpy(qw[1].copy())
    dkw = gpu.DeviceBuffer.from_numpy(kw[1].copy())
    start, n = 150, 400
    kc, vc = filled_cache(O, cfg, start, rng)
    q = normal_f32(rng, (n, cfg.q_dim), 3.0)
    k = normal_f32(rng, (n, cfg.kv_dim), 3.0)
    v = normal_f32(rng, (n, cfg.kv_dim))
    print(f"[case] prefill qknorm split {dims} start {start} n {n} tuning {tuning}", flush=True)
    cache = gpu.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = gpu.DeviceBuffer(n * cfg.q_dim * 4)
    gpu.check(gpu.lib.plh_set_tuning(*tuning), "plh_set_tuning")
    try:
        gpu.prefill(cache, 1, start, n, dq.ptr, dk.ptr, dv.ptr, dout.ptr, None, 1,
                    q_norm=dqw.ptr, k_norm=dkw.ptr, norm_eps=EPS)
        gpu.synchronize()
    finally:
        gpu.lib.plh_set_tuning(tuning[0], 0)
    out = dout.download(np.float32, (n, cfg.q_dim))
    gk, gv = cache.fetch()
    cache.free()
    shp = O.Shape(L, Hq, Hkv, D, S, theta, rt)
    cos_t, sin_t = O.rope_tables(S, D, theta)
    ref = O.attn_prefill(shp, 1, start, n, q.copy(), k.copy(), v, kc, vc, cos_t, sin_t,
                         q_norm=qw[1], k_norm=kw[1], eps=EPS)
    assert_attn_close(out, ref, D, what="prefill qknorm split layer 1")
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)
