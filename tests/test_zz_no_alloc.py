"""plh_attn_decode_noalloc (the allocation-free decode entry point) on the GPU.

Called through the C ABI and checked against plh_attn_decode on the same
inputs (outputs and appended cache rows bit-identical: same kernels, same
split plan, only the partials' storage differs) and against the oracle's
tolerance, on two calls in a row -- the second with a smaller input, which
reuses the static scratch holding the first call's partials.  A launch whose
partials would not fit in the static scratch is refused with -1 and a
message before anything runs."""
import numpy as np
import pytest

from attn_check import assert_attn_close, filled_cache, normal_f32

pytestmark = pytest.mark.gpu


def decode_call(P, fn, cfg, pos, q, k, v, kc, vc, n_layers):
    cache = P.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (P.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = P.DeviceBuffer(n_layers * cfg.q_dim * 4)
    dout.zero()
    rc = fn(cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
            cfg.rope_type, 0, n_layers, pos, dq.ptr, dk.ptr, dv.ptr, cache.key.ptr, cache.val.ptr,
            cache.cos.ptr, cache.sin.ptr, dout.ptr)
    P.synchronize()
    out = dout.download(np.float32, (n_layers, cfg.q_dim))
    gk, gv = cache.fetch()
    cache.free()
    return rc, out, gk, gv


CASES = [
    # (L, Hq, Hkv, D, S, theta, rope), pos: the first splits 22 layers of
    # 2047 rows, the second (smaller) 3 layers of 900 rows
    ((22, 32, 4, 64, 2048, 1e4, 0), 2047),
    ((3, 16, 8, 128, 1024, 1e6, 1), 900),
]


def test_noalloc_matches_decode_twice(gpu, oracle_mod):
    O = oracle_mod
    P = gpu
    for i, (dims, pos) in enumerate(CASES):
        cfg = P.AttnConfig(*dims)
        rng = np.random.default_rng(100 + i)
        kc, vc = filled_cache(O, cfg, pos, rng)
        q = normal_f32(rng, (cfg.n_layers, cfg.q_dim))
        k = normal_f32(rng, (cfg.n_layers, cfg.kv_dim))
        v = normal_f32(rng, (cfg.n_layers, cfg.kv_dim))
        print(f"[case] noalloc call {i}: {dims} pos {pos}", flush=True)
        rc_n, out_n, gk_n, gv_n = decode_call(P, P.lib.plh_attn_decode_noalloc, cfg, pos, q, k,
                                              v, kc, vc, cfg.n_layers)
        assert rc_n == 0, P._native.last_error()
        rc_d, out_d, gk_d, gv_d = decode_call(P, P.lib.plh_attn_decode, cfg, pos, q, k, v, kc,
                                              vc, cfg.n_layers)
        assert rc_d == 0
        assert np.array_equal(out_n.view(np.uint32), out_d.view(np.uint32))
        assert np.array_equal(gk_n, gk_d) and np.array_equal(gv_n, gv_d)
        shp = O.Shape(cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
                      cfg.rope_freq_base, cfg.rope_type)
        cos_t, sin_t = O.rope_tables(cfg.max_seq_len, cfg.head_dim, cfg.rope_freq_base)
        for l in (0, cfg.n_layers - 1):
            ref = O.attn_decode(shp, l, pos, q[l].copy(), k[l].copy(), v[l], kc, vc, cos_t,
                                sin_t)
            assert_attn_close(out_n[l], ref, cfg.head_dim, 1e-3, f"noalloc call {i} layer {l}")


def test_noalloc_captured_in_graph_from_fresh_library(gpu, oracle_mod):
    """The property the entry point exists for: it queues no allocation.
    The library is shut down and re-initialised so that no workspace
    exists, then a split launch (22 layers, pos 2047) is captured in a HIP
    graph before any allocating decode call (an allocation during capture
    fails the capture).  The graph is replayed three times with eager work
    and synchronisations between the replays; every replay's output and
    cache must equal an eager plh_attn_decode call bit for bit."""
    O, P = oracle_mod, gpu
    P.lib.plh_shutdown()
    P.init(0)
    cfg = P.AttnConfig(22, 32, 4, 64, 2048, 1e4, 0)
    pos = 2047
    rng = np.random.default_rng(300)
    kc, vc = filled_cache(O, cfg, pos, rng)
    q = normal_f32(rng, (cfg.n_layers, cfg.q_dim))
    k = normal_f32(rng, (cfg.n_layers, cfg.kv_dim))
    v = normal_f32(rng, (cfg.n_layers, cfg.kv_dim))
    cache = P.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (P.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = P.DeviceBuffer(cfg.n_layers * cfg.q_dim * 4)
    dout.zero()
    P.synchronize()
    args = (cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
            cfg.rope_type, 0, cfg.n_layers, pos, dq.ptr, dk.ptr, dv.ptr, cache.key.ptr,
            cache.val.ptr, cache.cos.ptr, cache.sin.ptr, dout.ptr)
    print("[case] noalloc captured from a fresh library", flush=True)
    with P.Graph() as g:
        P.check(P.lib.plh_attn_decode_noalloc(*args), "plh_attn_decode_noalloc (captured)")
    try:
        rc, want, wk, wv = decode_call(P, P.lib.plh_attn_decode, cfg, pos, q, k, v, kc, vc,
                                       cfg.n_layers)
        assert rc == 0
        for rep in range(3):
            dout.zero()
            cache.load(kc, vc)
            P.synchronize()
            g.launch()
            P.synchronize()
            got = dout.download(np.float32, (cfg.n_layers, cfg.q_dim))
            gk, gv = cache.fetch()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
            assert np.array_equal(gk, wk) and np.array_equal(gv, wv), rep
            # eager work between replays: an allocating call of another shape
            rc, _, _, _ = decode_call(P, P.lib.plh_attn_decode, P.AttnConfig(*CASES[1][0]),
                                      CASES[1][1], *small_inputs(O, P, rep), 3)
            assert rc == 0
    finally:
        cache.free()


def small_inputs(O, P, seed):
    cfg = P.AttnConfig(*CASES[1][0])
    rng = np.random.default_rng(400 + seed)
    kc, vc = filled_cache(O, cfg, CASES[1][1], rng)
    return (normal_f32(rng, (cfg.n_layers, cfg.q_dim)), normal_f32(rng, (cfg.n_layers, cfg.kv_dim)),
            normal_f32(rng, (cfg.n_layers, cfg.kv_dim)), kc, vc)


def test_noalloc_refuses_oversized_partials(gpu, oracle_mod):
    """8 layers x 8 kv heads x 16 q heads each, head_dim 128, 4095 cached
    rows, with tuning keys 1 and 8 asking for as many workgroups as the
    rows allow: the stream-K plan gives every 16-row block a workgroup of
    its own, 64 groups x 257 partial slots x 16 heads x 132 floats = 139 MB
    of partials (the split plan, 128-row splits, 17 MB), more than the
    static scratch holds.  The call returns -1 with a message and writes
    nothing; the workspace entry point runs the same launch."""
    P = gpu
    cfg = P.AttnConfig(8, 128, 8, 128, 4096, 1e4, 0)
    pos = 4095
    rng = np.random.default_rng(7)
    kc = np.zeros(cfg.cache_elems, np.uint16)
    vc = np.zeros(cfg.cache_elems, np.uint16)
    q = normal_f32(rng, (cfg.n_layers, cfg.q_dim))
    k = normal_f32(rng, (cfg.n_layers, cfg.kv_dim))
    v = normal_f32(rng, (cfg.n_layers, cfg.kv_dim))
    P.check(P.lib.plh_set_tuning(1, 1 << 20), "plh_set_tuning")   # split kernel
    P.check(P.lib.plh_set_tuning(8, 1 << 20), "plh_set_tuning")   # stream-K kernel
    try:
        print("[case] noalloc oversized partials", flush=True)
        rc, out, gk, gv = decode_call(P, P.lib.plh_attn_decode_noalloc, cfg, pos, q, k, v, kc,
                                      vc, cfg.n_layers)
        assert rc == -1
        assert "static scratch" in P._native.last_error()
        assert not out.any() and not gk.any() and not gv.any()
        rc, out, gk, gv = decode_call(P, P.lib.plh_attn_decode, cfg, pos, q, k, v, kc, vc,
                                      cfg.n_layers)
        assert rc == 0 and np.all(np.isfinite(out))
    finally:
        P.check(P.lib.plh_set_tuning(1, 0), "plh_set_tuning")
        P.check(P.lib.plh_set_tuning(8, 0), "plh_set_tuning")
