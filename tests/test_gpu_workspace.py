"""A graph captured before the decode workspace grows keeps replaying.

plh_attn_decode keeps its split partials in a library workspace that is
replaced by a larger one when a launch needs more.  A graph captured earlier
holds the old workspace's address in its kernel nodes, so an outgrown
workspace stays allocated until plh_shutdown.  The test captures a split
decode (2 TinyLlama-shaped layers at pos 2047) on a freshly initialised
library, grows the workspace with a launch whose split partials are many
times larger, then allocates and fills new buffers -- which could be placed
in the old workspace's memory had it been freed -- and replays the graph
three times: every replay's output and cache rows must equal the eager
call's bit for bit, and the new buffers must keep their contents."""
import numpy as np
import pytest

from attn_check import filled_cache, normal_f32

pytestmark = pytest.mark.gpu


def test_graph_replays_after_workspace_growth(gpu, oracle_mod):
    P, O = gpu, oracle_mod
    P.lib.plh_shutdown()
    P.init(0)
    cfg = P.AttnConfig(2, 32, 4, 64, 2048, 1e4, 0)
    pos = 2047
    rng = np.random.default_rng(500)
    kc, vc = filled_cache(O, cfg, pos, rng)
    q = normal_f32(rng, (cfg.n_layers, cfg.q_dim))
    k = normal_f32(rng, (cfg.n_layers, cfg.kv_dim))
    v = normal_f32(rng, (cfg.n_layers, cfg.kv_dim))
    cache = P.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (P.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = P.DeviceBuffer(cfg.n_layers * cfg.q_dim * 4)
    args = lambda out: (cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,  # noqa: E731
                        cfg.max_seq_len, cfg.rope_type, 0, cfg.n_layers, pos, dq.ptr, dk.ptr,
                        dv.ptr, cache.key.ptr, cache.val.ptr, cache.cos.ptr, cache.sin.ptr, out)
    big = None
    fresh = []
    try:
        print("[case] eager decode sizing the workspace", flush=True)
        P.check(P.lib.plh_attn_decode(*args(dout.ptr)), "plh_attn_decode")
        P.synchronize()
        want = dout.download(np.float32, (cfg.n_layers, cfg.q_dim))
        wk, wv = cache.fetch()
        gout = P.DeviceBuffer(cfg.n_layers * cfg.q_dim * 4)
        with P.Graph() as g:
            P.check(P.lib.plh_attn_decode(*args(gout.ptr)), "plh_attn_decode (captured)")
        # a launch with ~17 MB of split partials (the split kernel with as
        # many splits as the rows allow): the workspace is replaced
        print("[case] growing the workspace", flush=True)
        P.check(P.lib.plh_set_tuning(7, 1), "plh_set_tuning")
        P.check(P.lib.plh_set_tuning(1, 1 << 20), "plh_set_tuning")
        bcfg = P.AttnConfig(8, 128, 8, 128, 4096, 1e4, 0)
        big = P.KVCache(bcfg)
        big.load(np.zeros(bcfg.cache_elems, np.uint16), np.zeros(bcfg.cache_elems, np.uint16))
        bq = P.DeviceBuffer.from_numpy(normal_f32(rng, (bcfg.n_layers, bcfg.q_dim)))
        bk = P.DeviceBuffer.from_numpy(normal_f32(rng, (bcfg.n_layers, bcfg.kv_dim)))
        bo = P.DeviceBuffer(bcfg.n_layers * bcfg.q_dim * 4)
        P.check(P.lib.plh_attn_decode(bcfg.n_layers, bcfg.n_heads, bcfg.n_kv_heads,
                                      bcfg.head_dim, bcfg.max_seq_len, bcfg.rope_type, 0,
                                      bcfg.n_layers, 4095, bq.ptr, bk.ptr, bk.ptr, big.key.ptr,
                                      big.val.ptr, big.cos.ptr, big.sin.ptr, bo.ptr),
                "plh_attn_decode (large)")
        P.synchronize()
        # new allocations that a freed workspace's memory could serve
        for i in range(8):
            b = P.DeviceBuffer(1 << 20)
            b.upload(np.full(1 << 18, 0x5A5A0000 + i, np.uint32))
            fresh.append(b)
        P.synchronize()
        for rep in range(3):
            gout.zero()
            cache.load(kc, vc)
            P.synchronize()
            print(f"[case] replay {rep}", flush=True)
            g.launch()
            P.synchronize()
            got = gout.download(np.float32, (cfg.n_layers, cfg.q_dim))
            gk, gv = cache.fetch()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
            assert np.array_equal(gk, wk) and np.array_equal(gv, wv), rep
            for i, b in enumerate(fresh):
                assert np.all(b.download(np.uint32, (1 << 18,)) == 0x5A5A0000 + i), (rep, i)
    finally:
        P.check(P.lib.plh_set_tuning(7, 0), "plh_set_tuning")
        P.check(P.lib.plh_set_tuning(1, 0), "plh_set_tuning")
        cache.free()
        if big is not None:
            big.free()
        for b in fresh:
            b.free()
