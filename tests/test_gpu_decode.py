"""GPU parity of the decode path (plh_attn_decode) against the oracle.

Each case fills the FP16 caches with seeded N(0,1) rows 0..pos-1 (rounded by
the reference's fp32_to_fp16), runs one decode step on the device, and checks
  * every attention output head against the oracle (tolerance in attn_check),
  * the whole K and V caches bit for bit (row pos appended, nothing else
    touched).
Full-size configurations are checked on all layers where the oracle is fast
and on a sample of layers otherwise.
"""
import numpy as np
import pytest

from attn_check import assert_attn_close, filled_cache, normal_f32, tol_for

pytestmark = pytest.mark.gpu


def run_decode(P, O, cfg, pos, seed, check_layers=None, per_layer=False, poison=False,
               layer_range=None):
    rng = np.random.default_rng(seed)
    L = cfg.n_layers
    l0, nl = layer_range if layer_range else (0, L)
    kc, vc = filled_cache(O, cfg, pos, rng, poison_after=poison)
    q = normal_f32(rng, (nl, cfg.q_dim))
    k = normal_f32(rng, (nl, cfg.kv_dim))
    v = normal_f32(rng, (nl, cfg.kv_dim))
    print(f"[case] L{L} Hq{cfg.n_heads} Hkv{cfg.n_kv_heads} D{cfg.head_dim} S{cfg.max_seq_len} "
          f"pos {pos} layers [{l0},{l0 + nl}) per_layer={per_layer} seed {seed}", flush=True)
    cache = P.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (P.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = P.DeviceBuffer(nl * cfg.q_dim * 4)
    if per_layer:
        for i in range(nl):
            P.decode(cache, l0 + i, pos, dq.ptr + i * cfg.q_dim * 4, dk.ptr + i * cfg.kv_dim * 4,
                     dv.ptr + i * cfg.kv_dim * 4, dout.ptr + i * cfg.q_dim * 4, 1)
    else:
        P.decode(cache, l0, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, nl)
    P.synchronize()
    out = dout.download(np.float32, (nl, cfg.q_dim))
    gk, gv = cache.fetch()
    cache.free()

    shp = O.Shape(L, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.max_seq_len,
                  cfg.rope_freq_base, cfg.rope_type)
    cos_t, sin_t = O.rope_tables(cfg.max_seq_len, cfg.head_dim, cfg.rope_freq_base)
    rk, rv = kc.copy(), vc.copy()
    layers = range(nl) if check_layers is None else check_layers
    for i in range(nl):
        # every launched layer appends its row; the oracle appends it too
        lay = l0 + i
        qi, ki = q[i].copy(), k[i].copy()
        if i in layers:
            ref = O.attn_decode(shp, lay, pos, qi, ki, v[i], rk, rv, cos_t, sin_t)
            assert_attn_close(out[i], ref, cfg.head_dim, tol_for(pos + 1), f"layer {lay}")
        else:
            O.rope(qi, ki, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads, cos_t[pos], sin_t[pos],
                   cfg.rope_type)
            base = (lay * cfg.max_seq_len + pos) * cfg.kv_dim
            rk[base:base + cfg.kv_dim] = O.f32_to_f16(ki)
            rv[base:base + cfg.kv_dim] = O.f32_to_f16(v[i])
    bad_k = np.nonzero(gk != rk)[0]
    bad_v = np.nonzero(gv != rv)[0]
    assert bad_k.size == 0, f"K cache differs at {bad_k[:8]}"
    assert bad_v.size == 0, f"V cache differs at {bad_v[:8]}"
    return out


def test_layout_probe_fp16_exhaustive(gpu, oracle_mod):
    """All 2^32 fp32 inputs of the device fp32->fp16 rounding against the
    oracle (pinned to the reference's quant.c), in 16 checksummed slices."""
    chunk = 1 << 28
    for c in range(16):
        g = gpu.f16_checksum(c * chunk, chunk)
        o = oracle_mod.lib().orc_f16_checksum(c * chunk, chunk, 16)
        assert g == o, f"slice {c}: device {g:#x} oracle {o:#x}"


def test_f32_to_f16_array(gpu, oracle_mod):
    rng = np.random.default_rng(0)
    x = np.concatenate([normal_f32(rng, 100000), normal_f32(rng, 1000, 7e4),
                        normal_f32(rng, 1000, 1e-6),
                        np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 65520.0, 2.0 ** -25],
                                 np.float32)])
    d = gpu.DeviceBuffer.from_numpy(x)
    h = gpu.DeviceBuffer(x.size * 2)
    gpu.f32_to_f16(d.ptr, h.ptr, x.size)
    got = h.download(np.uint16, x.shape)
    assert np.array_equal(got, oracle_mod.f32_to_f16(x))


@pytest.mark.parametrize("path", ["decode_gqa4_d64.npz", "decode_gqa4_d128.npz",
                                  "decode_mha_qwen_d64.npz"])
def test_decode_replays_reference_golden(gpu, oracle_mod, path):
    """The reference's own outputs and caches (tests/golden), one token and
    one layer per call, as model_forward_ex issues them."""
    import os
    from conftest import GOLDEN
    z = np.load(os.path.join(GOLDEN, path))
    L, Hq, Hkv, D, S, rt = [int(x) for x in z["dims"]]
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, float(z["base"]), rt)
    cache = gpu.KVCache(cfg)
    dq = gpu.DeviceBuffer(cfg.q_dim * 4)
    dk = gpu.DeviceBuffer(cfg.kv_dim * 4)
    dv = gpu.DeviceBuffer(cfg.kv_dim * 4)
    dout = gpu.DeviceBuffer(cfg.q_dim * 4)
    q, k, v, want = z["q"], z["k"], z["v"], z["out"]
    for pos in range(q.shape[0]):
        for l in range(L):
            dq.upload(q[pos, l])
            dk.upload(k[pos, l])
            dv.upload(v[pos, l])
            gpu.decode(cache, l, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, 1)
            got = dout.download(np.float32, (cfg.q_dim,))
            assert_attn_close(got, want[pos, l], D, 1e-3, f"{path} pos {pos} layer {l}")
    gk, gv = cache.fetch()
    assert np.array_equal(gk, z["key_cache"]) and np.array_equal(gv, z["val_cache"])


# shapes of the three model families at small sizes, then edge positions
SMALL = [
    # (n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, theta, rope_type, pos)
    (2, 32, 4, 64, 512, 1e4, 0, 0),       # pos 0: only the appended row
    (2, 32, 4, 64, 512, 1e4, 0, 1),
    (2, 32, 4, 64, 512, 1e4, 0, 31),
    (2, 32, 4, 64, 512, 1e4, 0, 127),     # split boundaries (splits of 128 rows)
    (2, 32, 4, 64, 512, 1e4, 0, 128),
    (2, 32, 4, 64, 512, 1e4, 0, 129),
    (2, 32, 4, 64, 512, 1e4, 0, 511),     # last row of the cache
    (2, 32, 8, 64, 300, 5e5, 0, 299),     # Llama-3.2 head layout
    (2, 32, 32, 128, 260, 1e4, 0, 259),   # Llama-2 MHA, D=128
    (1, 16, 1, 64, 200, 1e4, 0, 150),     # G = 16
    (1, 32, 1, 64, 200, 1e4, 0, 150),     # G = 32: two q-head blocks per kv head
    (1, 12, 2, 64, 100, 1e4, 0, 70),      # G = 6
    (2, 8, 2, 64, 100, 1e4, 1, 70),       # QWEN rotation, D=64
    (2, 8, 2, 128, 100, 1e6, 1, 99),      # QWEN rotation, D=128
]


@pytest.mark.parametrize("case", SMALL)
def test_decode_small(gpu, oracle_mod, case):
    L, Hq, Hkv, D, S, theta, rt, pos = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    run_decode(gpu, oracle_mod, cfg, pos, seed=pos + 7 * D + Hkv)


def test_decode_per_layer_calls_equal_all_layer_launch(gpu, oracle_mod):
    cfg = gpu.AttnConfig(4, 32, 4, 64, 700, 1e4, 0)
    a = run_decode(gpu, oracle_mod, cfg, 600, seed=3, per_layer=True)
    b = run_decode(gpu, oracle_mod, cfg, 600, seed=3, per_layer=False)
    # both are checked against the oracle; split plans differ, so only close
    assert np.allclose(a, b, rtol=1e-4, atol=1e-6)


def test_decode_layer_subrange(gpu, oracle_mod):
    cfg = gpu.AttnConfig(6, 32, 4, 64, 300, 1e4, 0)
    run_decode(gpu, oracle_mod, cfg, 200, seed=5, layer_range=(2, 3))


def test_decode_ignores_rows_past_pos(gpu, oracle_mod):
    """Rows > pos hold NaN: the output must not see them (model.c:859 bound)."""
    cfg = gpu.AttnConfig(2, 32, 4, 64, 400, 1e4, 0)
    run_decode(gpu, oracle_mod, cfg, 257, seed=9, poison=True)


def test_decode_repeated_launches_keep_counters_clean(gpu, oracle_mod):
    """Different split plans back to back on one workspace."""
    for pos in (1000, 130, 2047, 5, 1500):
        cfg = gpu.AttnConfig(3, 32, 4, 64, 2048, 1e4, 0)
        run_decode(gpu, oracle_mod, cfg, pos, seed=pos, check_layers=[0, 2])


def test_decode_rejects_bad_arguments_without_side_effects(gpu, oracle_mod):
    cfg = gpu.AttnConfig(2, 32, 4, 64, 64, 1e4, 0)
    cache = gpu.KVCache(cfg)
    before = cache.fetch()
    buf = gpu.DeviceBuffer(cfg.q_dim * 4 * 2)
    for kwargs in ({"pos": 64}, {"pos": -1}):
        with pytest.raises(gpu.PicolmHipError):
            gpu.decode(cache, 0, kwargs["pos"], buf.ptr, buf.ptr, buf.ptr, buf.ptr, 1)
    with pytest.raises(gpu.PicolmHipError):
        gpu.decode(cache, 1, 3, buf.ptr, buf.ptr, buf.ptr, buf.ptr, 2)   # layers 1..2 of 2
    rc = gpu.lib.plh_attn_decode(2, 32, 4, 95, 64, 0, 0, 1, 0, buf.ptr, buf.ptr, buf.ptr,
                                 cache.key.ptr, cache.val.ptr, cache.cos.ptr, cache.sin.ptr,
                                 buf.ptr)                                 # odd head_dim
    assert rc == -1 and "head_dim" in gpu._native.last_error()
    gpu.synchronize()
    after = cache.fetch()
    assert np.array_equal(before[0], after[0]) and np.array_equal(before[1], after[1])


# ---- full-size configurations ------------------------------------------------

def test_cfg1_tinyllama_pos256(gpu, oracle_mod):
    cfg = gpu.AttnConfig(22, 32, 4, 64, 2048, 1e4, 0)
    run_decode(gpu, oracle_mod, cfg, 256, seed=101)


def test_cfg2_tinyllama_pos2047(gpu, oracle_mod):
    cfg = gpu.AttnConfig(22, 32, 4, 64, 2048, 1e4, 0)
    run_decode(gpu, oracle_mod, cfg, 2047, seed=102)


def test_cfg4_llama32_pos8191(gpu, oracle_mod):
    cfg = gpu.AttnConfig(16, 32, 8, 64, 8192, 5e5, 0)
    run_decode(gpu, oracle_mod, cfg, 8191, seed=104, check_layers=[0, 7, 15])


def test_cfg5a_llama2_pos4095(gpu, oracle_mod):
    cfg = gpu.AttnConfig(32, 32, 32, 128, 4096, 1e4, 0)
    run_decode(gpu, oracle_mod, cfg, 4095, seed=105, check_layers=[0, 31])


def test_decode_graph_replays_match_eager(gpu, oracle_mod):
    """A captured decode step (main + combine kernels) replayed several times,
    with eager work and synchronisation in between, gives the eager result
    each time."""
    cfg = gpu.AttnConfig(3, 32, 4, 64, 1024, 1e4, 0)
    rng = np.random.default_rng(21)
    pos = 900
    kc, vc = filled_cache(oracle_mod, cfg, pos, rng)
    q = normal_f32(rng, (3, cfg.q_dim))
    k = normal_f32(rng, (3, cfg.kv_dim))
    v = normal_f32(rng, (3, cfg.kv_dim))
    cache = gpu.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = gpu.DeviceBuffer(3 * cfg.q_dim * 4)
    gpu.decode(cache, 0, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, 3)
    gpu.synchronize()
    eager = dout.download(np.float32, (3, cfg.q_dim))
    with gpu.Graph() as g:
        gpu.decode(cache, 0, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, 3)
    scratch = gpu.DeviceBuffer(1 << 20)
    other = gpu.KVCache(cfg)          # eager work goes to a different cache
    other.load(kc, vc)
    for rep in range(4):
        dout.zero()
        scratch.zero()
        gpu.synchronize()
        g.launch()
        gpu.synchronize()
        got = dout.download(np.float32, (3, cfg.q_dim))
        assert np.array_equal(got, eager), f"replay {rep} differs from eager"
        # eager work between replays, with its own split plan and workspace use
        gpu.decode(other, 0, pos - 300, dq.ptr, dk.ptr, dv.ptr, scratch.ptr, 3)
    gk, gv = cache.fetch()
    assert np.array_equal(gk.reshape(3, -1, cfg.kv_dim)[:, :pos],
                          kc.reshape(3, -1, cfg.kv_dim)[:, :pos])


@pytest.mark.parametrize("workgroups", [1, 3, 7, 64, 256, 1000])
def test_decode_stream_k_plans(gpu, oracle_mod, workgroups):
    """Stream-K plans (plh_set_tuning key 8) from one workgroup walking every
    group whole (several groups per workgroup, no merge) to many short
    ranges (dozens of producers per group, merged in the kernel in batches
    of eight): oracle-exact outputs and caches, with ranges that start and
    end inside tiles, positions 0 and 1 (the new row only), a GQA group of
    24 q heads (two head blocks) and head_dim 128."""
    try:
        gpu.check(gpu.lib.plh_set_tuning(7, 2), "tuning")
        gpu.check(gpu.lib.plh_set_tuning(8, workgroups), "tuning")
        cfg = gpu.AttnConfig(4, 32, 4, 64, 2048, 1e4, 0)
        for pos in (2047, 700, 129, 17, 16, 1, 0):
            run_decode(gpu, oracle_mod, cfg, pos, seed=pos + workgroups, check_layers=[0, 3])
        cfg = gpu.AttnConfig(2, 32, 32, 128, 1024, 1e4, 0)
        run_decode(gpu, oracle_mod, cfg, 1000, seed=5 + workgroups)
        cfg = gpu.AttnConfig(2, 48, 2, 64, 600, 1e6, 1)
        run_decode(gpu, oracle_mod, cfg, 555, seed=6 + workgroups)
    finally:
        gpu.lib.plh_set_tuning(8, 0)
        gpu.lib.plh_set_tuning(7, 0)


@pytest.mark.parametrize("shape", [
    ((1, 32, 8, 64, 8192, 5e5, 0), 8191, 256),       # one Llama-3.2 layer: 32 producers a group
    ((2, 16, 8, 128, 4096, 1e6, 1), 2047, 256),      # head_dim 128, 16 producers a group
    ((22, 32, 4, 64, 2048, 1e4, 0), 2047, 256),      # TinyLlama, groups across XCD boundaries
    ((22, 32, 4, 64, 2048, 1e4, 0), 1024, 176),      # TinyLlama, two ranges a group (aligned)
    ((3, 48, 2, 64, 600, 1e4, 0), 599, 1000),        # two head blocks, 1000 workgroups
], ids=["llama32-layer", "d128", "tinyllama", "tinyllama-aligned", "hblk2-w1000"])
def test_decode_xcd_local_merges(gpu, oracle_mod, shape):
    """Stream-K merges inside one XCD's L2 (plh_set_tuning key 11 = 1) give
    oracle-exact outputs and caches, and the same bits as device-wide merges
    (key 11 = -1) under the same plan (workgroups fixed by key 8): the
    partials are merged in the same order either way."""
    dims, pos, workgroups = shape
    cfg = gpu.AttnConfig(*dims)
    check = None if cfg.n_layers <= 3 else [0, cfg.n_layers - 1]
    outs = {}
    try:
        gpu.check(gpu.lib.plh_set_tuning(7, 2), "tuning")
        gpu.check(gpu.lib.plh_set_tuning(8, workgroups), "tuning")
        for mode in (1, -1):
            gpu.check(gpu.lib.plh_set_tuning(11, mode), "tuning")
            outs[mode] = run_decode(gpu, oracle_mod, cfg, pos, seed=77, check_layers=check)
    finally:
        gpu.lib.plh_set_tuning(11, 0)
        gpu.lib.plh_set_tuning(8, 0)
        gpu.lib.plh_set_tuning(7, 0)
    assert np.array_equal(outs[1].view(np.uint32), outs[-1].view(np.uint32))


@pytest.mark.parametrize("shape", [
    ((1, 32, 4, 64, 2048, 1e4, 0), 530),    # one TinyLlama layer: 4 ranges a group, uneven
    ((1, 32, 4, 64, 2048, 1e4, 0), 700),    # 4 ranges of 11 blocks
    ((1, 32, 4, 64, 2048, 1e4, 0), 2047),   # 8 ranges of 16 blocks
    ((1, 24, 3, 64, 1024, 1e4, 0), 1000),   # 3 groups, 4 ranges of 15-16 blocks
    ((22, 32, 4, 64, 1024, 1e4, 0), 1000),  # 88 groups: the XCD-local aligned plan, uneven
], ids=["tl-530", "tl-700", "tl-2047", "3groups", "88groups"])
def test_decode_aligned_plans(gpu, oracle_mod, shape):
    """The default stream-K plans that give every group its own ranges
    (including group block counts the ranges do not divide evenly): oracle-
    exact outputs and caches."""
    dims, pos = shape
    try:
        gpu.check(gpu.lib.plh_set_tuning(7, 2), "tuning")
        run_decode(gpu, oracle_mod, gpu.AttnConfig(*dims), pos, seed=pos + dims[2])
    finally:
        gpu.lib.plh_set_tuning(7, 0)


@pytest.mark.parametrize("merge", [0, -1], ids=["in-launch", "combine"])
@pytest.mark.parametrize("min_split", [128, 512, 1024, 2048])
def test_decode_split_lengths(gpu, oracle_mod, min_split, merge):
    """The split kernel (plh_set_tuning key 7 = 1) under several split plans
    (one split included), its partials merged by the group's last split in
    the launch (key 14 = 0) or by the combine launch (key 14 = -1): oracle-
    exact results."""
    try:
        gpu.check(gpu.lib.plh_set_tuning(7, 1), "tuning")
        gpu.check(gpu.lib.plh_set_tuning(2, min_split), "tuning")
        gpu.check(gpu.lib.plh_set_tuning(14, merge), "tuning")
        cfg = gpu.AttnConfig(4, 32, 4, 64, 2048, 1e4, 0)
        for pos in (2047, 700, 129):
            run_decode(gpu, oracle_mod, cfg, pos, seed=pos + min_split, check_layers=[0, 3])
        cfg = gpu.AttnConfig(2, 32, 32, 128, 1024, 1e4, 0)
        run_decode(gpu, oracle_mod, cfg, 1000, seed=5 + min_split)
    finally:
        gpu.lib.plh_set_tuning(14, 0)
        gpu.lib.plh_set_tuning(2, 0)
        gpu.lib.plh_set_tuning(7, 0)
