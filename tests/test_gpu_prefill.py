"""GPU parity of the prefill path (plh_attn_prefill) against the oracle.

Each case fills the FP16 caches with seeded N(0,1) prefix rows 0..start-1
(what kvcache_load leaves, picolm.c:214-230), runs one prefill of n tokens
on the device, and checks
  * every token's attention output head against the oracle (tolerance in
    attn_check),
  * the whole K and V caches bit for bit (rows start..start+n-1 appended,
    nothing else touched).
"""
import os

import numpy as np
import pytest

from attn_check import assert_attn_close, filled_cache, normal_f32, tol_for

pytestmark = pytest.mark.gpu


def run_prefill(P, O, cfg, start, n, seed, check_layers=None, per_layer=False, out_stride=None,
                layer_range=None):
    rng = np.random.default_rng(seed)
    L = cfg.n_layers
    l0, nl = layer_range if layer_range else (0, L)
    stride = cfg.q_dim if out_stride is None else out_stride
    kc, vc = filled_cache(O, cfg, start, rng)
    q = normal_f32(rng, (nl, n, cfg.q_dim))
    k = normal_f32(rng, (nl, n, cfg.kv_dim))
    v = normal_f32(rng, (nl, n, cfg.kv_dim))
    print(f"[case] L{L} Hq{cfg.n_heads} Hkv{cfg.n_kv_heads} D{cfg.head_dim} S{cfg.max_seq_len} "
          f"start {start} n {n} layers [{l0},{l0 + nl}) per_layer={per_layer} stride {stride} "
          f"seed {seed}", flush=True)
    cache = P.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (P.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = P.DeviceBuffer(max(1, nl * n * stride * 4))
    dout.zero()
    if per_layer:
        for i in range(nl):
            P.prefill(cache, l0 + i, start, n, dq.ptr + i * n * cfg.q_dim * 4,
                      dk.ptr + i * n * cfg.kv_dim * 4, dv.ptr + i * n * cfg.kv_dim * 4,
                      dout.ptr + i * n * stride * 4, stride, 1)
    else:
        P.prefill(cache, l0, start, n, dq.ptr, dk.ptr, dv.ptr, dout.ptr, stride, nl)
    P.synchronize()
    out = dout.download(np.float32, (nl, n, stride)) if n else np.zeros((nl, 0, stride), np.float32)
    gk, gv = cache.fetch()
    cache.free()

    shp = O.Shape(L, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
                  cfg.rope_freq_base, cfg.rope_type)
    cos_t, sin_t = O.rope_tables(cfg.max_seq_len, cfg.head_dim, cfg.rope_freq_base)
    rk, rv = kc.copy(), vc.copy()
    layers = range(nl) if check_layers is None else check_layers
    for i in range(nl):
        lay = l0 + i
        if i in layers and n > 0:
            ref = O.attn_prefill(shp, lay, start, n, q[i].copy(), k[i].copy(), v[i], rk, rv,
                                 cos_t, sin_t)
            assert_attn_close(out[i, :, :cfg.q_dim], ref, cfg.head_dim, tol_for(start + n),
                              f"layer {lay}")
        else:
            ki = k[i].copy()
            for t in range(n):
                qq = np.zeros(cfg.q_dim, np.float32)
                O.rope(qq, ki[t], cfg.head_dim, cfg.n_heads, cfg.n_kv_heads, cos_t[start + t],
                       sin_t[start + t], cfg.rope_type)
            base = (lay * cfg.max_seq_len + start) * cfg.kv_dim
            rk[base:base + n * cfg.kv_dim] = O.f32_to_f16(ki.reshape(-1))
            rv[base:base + n * cfg.kv_dim] = O.f32_to_f16(v[i].reshape(-1))
    if stride > cfg.q_dim and n:
        assert np.all(out[:, :, cfg.q_dim:] == 0), "wrote past n_heads*head_dim"
    bad_k = np.nonzero(gk != rk)[0]
    bad_v = np.nonzero(gv != rv)[0]
    assert bad_k.size == 0, f"K cache differs at {bad_k[:8]}"
    assert bad_v.size == 0, f"V cache differs at {bad_v[:8]}"
    return out


@pytest.mark.parametrize("path", ["prefill_gqa4_d64.npz", "prefill_gqa4_d128.npz"])
def test_prefill_replays_reference_golden(gpu, oracle_mod, path):
    """The reference's own chunked prefill (second chunk attends over the
    first one's cached rows), one layer per call as model_forward_prefill
    issues them; outputs and final caches from tests/golden."""
    from conftest import GOLDEN
    z = np.load(os.path.join(GOLDEN, path))
    L, Hq, Hkv, D, S, rt = [int(x) for x in z["dims"]]
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, float(z["base"]), rt)
    cache = gpu.KVCache(cfg)
    start = 0
    for ci, n in enumerate(z["chunks"]):
        n = int(n)
        for l in range(L):
            dq = gpu.DeviceBuffer.from_numpy(z[f"q_{ci}_{l}"])
            dk = gpu.DeviceBuffer.from_numpy(z[f"k_{ci}_{l}"])
            dv = gpu.DeviceBuffer.from_numpy(z[f"v_{ci}_{l}"])
            dout = gpu.DeviceBuffer(n * cfg.q_dim * 4)
            gpu.prefill(cache, l, start, n, dq.ptr, dk.ptr, dv.ptr, dout.ptr)
            got = dout.download(np.float32, (n, cfg.q_dim))
            assert_attn_close(got, z[f"out_{ci}_{l}"], D, 1e-3, f"{path} chunk {ci} layer {l}")
        start += n
    gk, gv = cache.fetch()
    assert np.array_equal(gk, z["key_cache"]) and np.array_equal(gv, z["val_cache"])


SMALL = [
    # (n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, theta, rope_type, start, n)
    (2, 32, 4, 64, 256, 1e4, 0, 0, 1),        # one token
    (2, 32, 4, 64, 256, 1e4, 0, 0, 17),       # ragged last q block (bq = 16)
    (2, 32, 4, 64, 256, 1e4, 0, 0, 64),
    (2, 32, 4, 64, 256, 1e4, 0, 37, 50),      # prefix in the cache
    (2, 32, 4, 64, 256, 1e4, 0, 200, 56),     # ends on the last cache row
    (2, 32, 8, 64, 300, 5e5, 0, 0, 100),      # Llama-3.2 heads, G = 4
    (2, 32, 32, 128, 300, 1e4, 0, 0, 130),    # Llama-2 MHA, D = 128
    (2, 32, 32, 128, 300, 1e4, 0, 99, 70),    # MHA with prefix
    (1, 16, 1, 64, 200, 1e4, 0, 5, 40),       # G = 16
    (1, 32, 1, 64, 200, 1e4, 0, 5, 40),       # G = 32
    (1, 12, 2, 64, 100, 1e4, 0, 3, 33),       # G = 6 (columns not a multiple of G)
    (2, 8, 2, 64, 100, 1e4, 1, 10, 45),       # QWEN rotation, D = 64
    (2, 8, 2, 128, 100, 1e6, 1, 0, 31),       # QWEN rotation, D = 128
]


# launches whose heavy q blocks are split into chunks of tiles (partials merged
# afterwards): automatic for one-layer launches with few q blocks (a prompt
# chunk late in the prompt), forced here through plh_set_tuning key 5 for the
# other chunk sizes
SPLIT = [
    # (n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, theta, rope_type, start, n,
    #  layer, chunk tiles: 0 = automatic)
    (3, 32, 4, 64, 1024, 1e4, 0, 0, 512, 1, 4),     # TinyLlama heads, one layer of three
    (2, 32, 4, 64, 1024, 1e4, 0, 300, 333, 0, 2),   # prefix rows, ragged last block
    (2, 32, 8, 64, 800, 5e5, 0, 17, 700, 1, 16),    # Llama-3.2 heads
    (2, 32, 32, 128, 1100, 1e4, 0, 0, 1024, 0, 8),  # Llama-2 MHA, D = 128
    (2, 8, 2, 128, 700, 1e6, 1, 40, 600, 1, 0),     # QWEN rotation, D = 128 (automatic)
    (2, 32, 4, 64, 1200, 1e4, 0, 1024, 128, 1, 0),  # a 128-token chunk late in the prompt
]


@pytest.mark.parametrize("case", SPLIT)
def test_prefill_one_layer_split(gpu, oracle_mod, case):
    L, Hq, Hkv, D, S, theta, rt, start, n, layer, chunk = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    gpu.check(gpu.lib.plh_set_tuning(5, chunk), "plh_set_tuning")
    try:
        run_prefill(gpu, oracle_mod, cfg, start, n, seed=start + n + layer, check_layers=[0],
                    layer_range=(layer, 1))
    finally:
        gpu.lib.plh_set_tuning(5, 0)


@pytest.mark.parametrize("case", SMALL)
def test_prefill_small(gpu, oracle_mod, case):
    L, Hq, Hkv, D, S, theta, rt, start, n = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    run_prefill(gpu, oracle_mod, cfg, start, n, seed=start * 7 + n + D)


# K-split workgroups (2 or 3 groups of 4 waves share a q block's tiles and
# merge in LDS): automatic for one-layer launches of a whole prompt (more q
# blocks than a quarter of the CUs, at most one per CU), forced through
# plh_set_tuning key 6 otherwise (3 groups only for head_dim 64)
KSPLIT = [
    # (n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, theta, rope_type, start, n,
    #  layer, groups: 0 = automatic)
    (3, 32, 4, 64, 1024, 1e4, 0, 0, 512, 1, 0),     # TinyLlama heads: 128 q blocks
    (2, 32, 4, 64, 1024, 1e4, 0, 0, 512, 0, 2),     # the same, 2 groups
    (2, 32, 8, 64, 800, 5e5, 0, 0, 500, 1, 0),      # Llama-3.2 heads: 128 q blocks
    (2, 32, 32, 128, 1100, 1e4, 0, 0, 1024, 0, 0),  # Llama-2 MHA, D = 128: 256 q blocks
    (2, 32, 4, 64, 600, 1e4, 0, 37, 500, 0, 3),     # prefix rows, ragged last block
    (2, 8, 2, 128, 300, 1e6, 1, 10, 150, 1, 2),     # QWEN rotation, D = 128
]


@pytest.mark.parametrize("case", KSPLIT)
def test_prefill_one_layer_ksplit(gpu, oracle_mod, case):
    L, Hq, Hkv, D, S, theta, rt, start, n, layer, groups = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    gpu.check(gpu.lib.plh_set_tuning(6, groups), "plh_set_tuning")
    try:
        run_prefill(gpu, oracle_mod, cfg, start, n, seed=start + n + layer + 5,
                    check_layers=[0], layer_range=(layer, 1))
    finally:
        gpu.lib.plh_set_tuning(6, 0)


@pytest.mark.parametrize("groups", [2, 3])
@pytest.mark.parametrize("case", SMALL)
def test_prefill_small_ksplit(gpu, oracle_mod, case, groups):
    """Every small case through forced K-split workgroups (all layers in one
    launch; groups without a tile of their own, masked first tiles)."""
    L, Hq, Hkv, D, S, theta, rt, start, n = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    gpu.check(gpu.lib.plh_set_tuning(6, groups), "plh_set_tuning")
    try:
        run_prefill(gpu, oracle_mod, cfg, start, n, seed=start * 5 + n + D + groups)
    finally:
        gpu.lib.plh_set_tuning(6, 0)


def test_prefill_per_layer_and_all_layers(gpu, oracle_mod):
    cfg = gpu.AttnConfig(3, 32, 4, 64, 256, 1e4, 0)
    a = run_prefill(gpu, oracle_mod, cfg, 20, 70, seed=4, per_layer=True)
    b = run_prefill(gpu, oracle_mod, cfg, 20, 70, seed=4, per_layer=False)
    assert np.array_equal(a, b)


def test_prefill_layer_subrange_and_wide_stride(gpu, oracle_mod):
    """Layers [1, 3) of 4, output rows strided wider than n_heads*head_dim
    (the reference writes into xb_batch with stride n_embd)."""
    cfg = gpu.AttnConfig(4, 32, 4, 64, 128, 1e4, 0)
    run_prefill(gpu, oracle_mod, cfg, 9, 40, seed=5, layer_range=(1, 2),
                out_stride=cfg.q_dim + 64)


def test_prefill_split_wide_stride(gpu, oracle_mod):
    """A split one-layer launch (chunks of 2 tiles, merged) writing output rows
    strided wider than n_heads*head_dim: the merge kernel honours the stride
    and writes nothing past each row's heads."""
    cfg = gpu.AttnConfig(2, 32, 4, 64, 512, 1e4, 0)
    gpu.check(gpu.lib.plh_set_tuning(5, 2), "plh_set_tuning")
    try:
        run_prefill(gpu, oracle_mod, cfg, 60, 200, seed=12, layer_range=(1, 1),
                    out_stride=cfg.q_dim + 96)
    finally:
        gpu.lib.plh_set_tuning(5, 0)


def test_prefill_zero_tokens_is_a_no_op(gpu, oracle_mod):
    cfg = gpu.AttnConfig(2, 32, 4, 64, 64, 1e4, 0)
    run_prefill(gpu, oracle_mod, cfg, 10, 0, seed=6)


def test_prefill_rejects_bad_arguments_without_side_effects(gpu):
    cfg = gpu.AttnConfig(2, 32, 4, 64, 64, 1e4, 0)
    cache = gpu.KVCache(cfg)
    before = cache.fetch()
    buf = gpu.DeviceBuffer(64 * cfg.q_dim * 4)
    for start, n in ((60, 5), (-1, 3), (0, -2)):
        with pytest.raises(gpu.PicolmHipError):
            gpu.prefill(cache, 0, start, n, buf.ptr, buf.ptr, buf.ptr, buf.ptr)
    with pytest.raises(gpu.PicolmHipError):
        gpu.prefill(cache, 0, 0, 4, buf.ptr, buf.ptr, buf.ptr, buf.ptr, cfg.q_dim - 4)
    with pytest.raises(gpu.PicolmHipError):
        gpu.prefill(cache, 1, 0, 4, buf.ptr, buf.ptr, buf.ptr, buf.ptr, None, 2)
    gpu.synchronize()
    after = cache.fetch()
    assert np.array_equal(before[0], after[0]) and np.array_equal(before[1], after[1])


def test_prefill_then_decode_continues_the_sequence(gpu, oracle_mod):
    """Prefill rows 0..n-1 on the device, then decode at pos n over the device
    cache: the decode step matches the oracle run over the same history."""
    cfg = gpu.AttnConfig(2, 32, 4, 64, 512, 1e4, 0)
    rng = np.random.default_rng(8)
    n = 300
    q = normal_f32(rng, (2, n, cfg.q_dim))
    k = normal_f32(rng, (2, n, cfg.kv_dim))
    v = normal_f32(rng, (2, n, cfg.kv_dim))
    qd = normal_f32(rng, (2, cfg.q_dim))
    kd = normal_f32(rng, (2, cfg.kv_dim))
    vd = normal_f32(rng, (2, cfg.kv_dim))
    cache = gpu.KVCache(cfg)
    bufs = [gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v, qd, kd, vd)]
    pout = gpu.DeviceBuffer(2 * n * cfg.q_dim * 4)
    dout = gpu.DeviceBuffer(2 * cfg.q_dim * 4)
    gpu.prefill(cache, 0, 0, n, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, pout.ptr, None, 2)
    gpu.decode(cache, 0, n, bufs[3].ptr, bufs[4].ptr, bufs[5].ptr, dout.ptr, 2)
    gpu.synchronize()
    got = dout.download(np.float32, (2, cfg.q_dim))
    shp = oracle_mod.Shape(2, 32, 4, 64, 512)
    cos_t, sin_t = oracle_mod.rope_tables(512, 64, 1e4)
    kc = np.zeros(cfg.cache_elems, np.uint16)
    vc = kc.copy()
    for l in range(2):
        oracle_mod.attn_prefill(shp, l, 0, n, q[l].copy(), k[l].copy(), v[l], kc, vc, cos_t, sin_t)
        ref = oracle_mod.attn_decode(shp, l, n, qd[l].copy(), kd[l].copy(), vd[l], kc, vc,
                                     cos_t, sin_t)
        assert_attn_close(got[l], ref, 64, 1e-3, f"decode after prefill, layer {l}")
    gk, gv = cache.fetch()
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)


# ---- full-size configurations ------------------------------------------------

def test_cfg3_tinyllama_prefill_512(gpu, oracle_mod):
    cfg = gpu.AttnConfig(22, 32, 4, 64, 2048, 1e4, 0)
    run_prefill(gpu, oracle_mod, cfg, 0, 512, seed=103, check_layers=[0, 5, 11, 21])


def test_cfg5b_llama2_prefill_1024(gpu, oracle_mod):
    cfg = gpu.AttnConfig(32, 32, 32, 128, 4096, 1e4, 0)
    run_prefill(gpu, oracle_mod, cfg, 0, 1024, seed=106, check_layers=[0, 31])


def test_prefill_split_graph_replays_match_eager(gpu, oracle_mod):
    """A captured one-layer prefill that splits its heavy q blocks (attention
    chunks + merge kernel, partials in the library workspace) replayed several
    times, with eager prefill work in between, gives the eager result each
    time."""
    cfg = gpu.AttnConfig(2, 32, 4, 64, 1400, 1e4, 0)
    rng = np.random.default_rng(31)
    start, n = 1024, 128
    kc, vc = filled_cache(oracle_mod, cfg, start, rng)
    q = normal_f32(rng, (n, cfg.q_dim))
    k = normal_f32(rng, (n, cfg.kv_dim))
    v = normal_f32(rng, (n, cfg.kv_dim))
    cache = gpu.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = gpu.DeviceBuffer(n * cfg.q_dim * 4)
    gpu.prefill(cache, 1, start, n, dq.ptr, dk.ptr, dv.ptr, dout.ptr)
    gpu.synchronize()
    eager = dout.download(np.float32, (n, cfg.q_dim))
    with gpu.Graph() as g:
        gpu.prefill(cache, 1, start, n, dq.ptr, dk.ptr, dv.ptr, dout.ptr)
    other = gpu.KVCache(cfg)          # eager work goes to a different cache
    other.load(kc, vc)
    scratch = gpu.DeviceBuffer(n * cfg.q_dim * 4)
    for rep in range(4):
        dout.zero()
        gpu.synchronize()
        g.launch()
        gpu.synchronize()
        got = dout.download(np.float32, (n, cfg.q_dim))
        assert np.array_equal(got, eager), f"replay {rep} differs from eager"
        # eager split launches between replays reuse the same workspace
        gpu.prefill(other, 1, start - 200, n, dq.ptr, dk.ptr, dv.ptr, scratch.ptr)
    shp = oracle_mod.Shape(2, 32, 4, 64, 1400)
    cos_t, sin_t = oracle_mod.rope_tables(1400, 64, 1e4)
    ref = oracle_mod.attn_prefill(shp, 1, start, n, q.copy(), k.copy(), v, kc, vc, cos_t, sin_t)
    assert_attn_close(eager, ref, 64, 1e-3, "eager split prefill")
    gk, gv = cache.fetch()
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)
