"""Pins the oracle's attention block (model.c:802-892 decode, 1019-1090 prefill).

Checks, each chosen so that a plausible slip (wrong kv-head index, a missing
1/sqrt(D), a causal off-by-one, a transposed cache index) fails one of them:
  * replay of the reference's own outputs and caches (tests/golden/*.npz),
  * live comparison with the reference's model_forward_ex / _prefill when the
    harness is built,
  * a double-precision textbook softmax(q K^T / sqrt(D)) V on small inputs,
  * closed-form special cases.
"""
import glob
import os

import numpy as np
import pytest

from conftest import GOLDEN, needs_ref


def shape_from(z, O):
    L, Hq, Hkv, D, S, rt = [int(x) for x in z["dims"]]
    return O.Shape(L, Hq, Hkv, D, S, float(z["base"]), rt)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "decode_*.npz"))))
def test_decode_replays_reference(oracle_mod, path):
    O = oracle_mod
    z = np.load(path)
    shp = shape_from(z, O)
    c, s = O.rope_tables(shp.max_seq_len, shp.head_dim, shp.rope_base)
    kc = np.zeros(shp.cache_elems(), np.uint16)
    vc = kc.copy()
    q, k, v, want = z["q"], z["k"], z["v"], z["out"]
    for pos in range(q.shape[0]):
        for l in range(shp.n_layers):
            out = O.attn_decode(shp, l, pos, q[pos, l].copy(), k[pos, l].copy(),
                                np.ascontiguousarray(v[pos, l]), kc, vc, c, s)
            assert np.array_equal(out.view(np.uint32), want[pos, l].view(np.uint32)), (pos, l)
    assert np.array_equal(kc, z["key_cache"]) and np.array_equal(vc, z["val_cache"])


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "prefill_*.npz"))))
def test_prefill_replays_reference(oracle_mod, path):
    O = oracle_mod
    z = np.load(path)
    shp = shape_from(z, O)
    c, s = O.rope_tables(shp.max_seq_len, shp.head_dim, shp.rope_base)
    kc = np.zeros(shp.cache_elems(), np.uint16)
    vc = kc.copy()
    start = 0
    for ci, n in enumerate(z["chunks"]):
        for l in range(shp.n_layers):
            out = O.attn_prefill(shp, l, start, int(n), z[f"q_{ci}_{l}"].copy(),
                                 z[f"k_{ci}_{l}"].copy(), z[f"v_{ci}_{l}"], kc, vc, c, s)
            assert np.array_equal(out.view(np.uint32), z[f"out_{ci}_{l}"].view(np.uint32))
        start += int(n)
    assert np.array_equal(kc, z["key_cache"]) and np.array_equal(vc, z["val_cache"])


@needs_ref
@pytest.mark.parametrize("L,Hq,Hkv,D,S,base,rt", [
    (2, 32, 4, 64, 40, 1e4, 0),      # TinyLlama head layout, short cache
    (2, 8, 8, 128, 24, 1e4, 0),      # MHA, D=128 (Llama-2 head layout)
    (1, 8, 2, 64, 30, 5e5, 1),       # QWEN rotation
])
def test_decode_matches_reference_live(oracle_mod, L, Hq, Hkv, D, S, base, rt):
    O = oracle_mod
    shp = O.Shape(L, Hq, Hkv, D, S, base, rt)
    rm = O.RefModel(shp, 0, seed=3)
    R = O.ref()
    rng = np.random.default_rng(4)
    c, s = O.rope_tables(S, D, base)
    kc = np.zeros(shp.cache_elems(), np.uint16)
    vc = kc.copy()
    try:
        for pos in range(S):
            qs = (rng.standard_normal((L, shp.q_dim)) * 2).astype(np.float32)
            ks = (rng.standard_normal((L, shp.kv_dim)) * 2).astype(np.float32)
            vs = rng.standard_normal((L, shp.kv_dim)).astype(np.float32)
            for l in range(L):
                R.ref_set_decode_qkv(rm.h, l, qs[l], ks[l], vs[l])
            want = np.empty(shp.q_dim, np.float32)
            R.ref_decode(rm.h, pos, L, want)
            for l in range(L):
                out = O.attn_decode(shp, l, pos, qs[l].copy(), ks[l].copy(), vs[l], kc, vc, c, s)
            assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), pos
        assert np.array_equal(kc, rm.kc) and np.array_equal(vc, rm.vc)
    finally:
        rm.close()


def textbook(O, q, kc, vc, shp, layer, pos):
    """softmax(q K^T / sqrt(D)) V in float64 over rows 0..pos."""
    D, Hkv = shp.head_dim, shp.n_kv_heads
    G = shp.n_heads // Hkv
    kc, vc = O.f16_to_f32(kc), O.f16_to_f32(vc)
    K = kc.reshape(shp.n_layers, shp.max_seq_len, Hkv, D)[layer, : pos + 1]
    V = vc.reshape(shp.n_layers, shp.max_seq_len, Hkv, D)[layer, : pos + 1]
    out = np.empty((shp.n_heads, D))
    for h in range(shp.n_heads):
        sc = K[:, h // G, :].astype(np.float64) @ q[h * D:(h + 1) * D].astype(np.float64) / np.sqrt(D)
        w = np.exp(sc - sc.max())
        out[h] = (w @ V[:, h // G, :].astype(np.float64)) / w.sum()
    return out.reshape(-1)


def random_cache(O, shp, rng, scale=1.0):
    n = shp.cache_elems()
    kc = O.f32_to_f16((rng.standard_normal(n) * scale).astype(np.float32))
    vc = O.f32_to_f16(rng.standard_normal(n).astype(np.float32))
    return kc, vc


@pytest.mark.parametrize("Hq,Hkv,D,pos", [(8, 1, 64, 0), (8, 2, 64, 37), (4, 4, 128, 99), (6, 3, 32, 5)])
def test_decode_against_textbook_double(oracle_mod, Hq, Hkv, D, pos):
    O = oracle_mod
    shp = O.Shape(2, Hq, Hkv, D, 128)
    rng = np.random.default_rng(pos + D)
    kc, vc = random_cache(O, shp, rng, scale=2.0)
    q = (rng.standard_normal(shp.q_dim) * 2).astype(np.float32)
    out = O.attn_core(shp, 1, pos, q, kc, vc)
    ref = textbook(O, q, kc, vc, shp, 1, pos)
    assert np.max(np.abs(out - ref)) <= 2e-5 * np.max(np.abs(ref))


def test_pos0_returns_v0_exactly(oracle_mod):
    O = oracle_mod
    shp = O.Shape(1, 4, 2, 64, 8)
    rng = np.random.default_rng(1)
    kc, vc = random_cache(O, shp, rng)
    out = O.attn_core(shp, 0, 0, rng.standard_normal(shp.q_dim).astype(np.float32), kc, vc)
    v0 = O.f16_to_f32(vc[: shp.kv_dim]).reshape(2, 64)
    assert np.array_equal(out.reshape(4, 64), np.repeat(v0, 2, axis=0))


def test_identical_keys_average_values(oracle_mod):
    O = oracle_mod
    shp = O.Shape(1, 2, 1, 64, 300)
    rng = np.random.default_rng(2)
    _, vc = random_cache(O, shp, rng)
    kc = np.tile(O.f32_to_f16(rng.standard_normal(64).astype(np.float32)), 300)
    out = O.attn_core(shp, 0, 299, rng.standard_normal(128).astype(np.float32), kc, vc)
    mean = O.f16_to_f32(vc).reshape(300, 64).astype(np.float64).mean(0)
    assert np.max(np.abs(out.reshape(2, 64) - mean)) < 1e-5


def test_dominant_score_selects_its_row(oracle_mod):
    O = oracle_mod
    shp = O.Shape(1, 1, 1, 64, 50)
    rng = np.random.default_rng(3)
    kc, vc = random_cache(O, shp, rng, scale=0.01)
    q = np.zeros(64, np.float32)
    q[5] = 1000.0
    kc.reshape(50, 64)[17, 5] = O.f32_to_f16(np.array([10.0], np.float32))[0]
    out = O.attn_core(shp, 0, 49, q, kc, vc)
    assert np.array_equal(out, O.f16_to_f32(vc.reshape(50, 64)[17]))


def test_gqa_head_mapping(oracle_mod):
    """Constant, distinct V per kv head: q head h must return kv head h // G."""
    O = oracle_mod
    Hq, Hkv, D, S = 12, 3, 32, 20
    shp = O.Shape(1, Hq, Hkv, D, S)
    rng = np.random.default_rng(4)
    kc, _ = random_cache(O, shp, rng)
    v = np.zeros((S, Hkv, D), np.float32)
    for j in range(Hkv):
        v[:, j, :] = j + 1
    vc = O.f32_to_f16(v.reshape(-1))
    out = O.attn_core(shp, 0, S - 1, rng.standard_normal(Hq * D).astype(np.float32), kc, vc)
    for h in range(Hq):
        assert np.allclose(out[h * D:(h + 1) * D], h // (Hq // Hkv) + 1, rtol=1e-6, atol=0)


def test_rows_after_pos_are_not_read(oracle_mod):
    O = oracle_mod
    shp = O.Shape(2, 8, 2, 64, 64)
    rng = np.random.default_rng(5)
    kc, vc = random_cache(O, shp, rng)
    q = rng.standard_normal(shp.q_dim).astype(np.float32)
    a = O.attn_core(shp, 1, 30, q, kc, vc)
    kc2, vc2 = kc.copy(), vc.copy()
    for cache in (kc2, vc2):
        c = cache.reshape(2, 64, shp.kv_dim)
        c[1, 31:] = 0x7E00          # NaN rows beyond pos
        c[0] = 0x7E00               # and the other layer
    b = O.attn_core(shp, 1, 30, q, kc2, vc2)
    assert np.array_equal(a, b)


def test_prefill_equals_sequential_decode(oracle_mod):
    O = oracle_mod
    shp = O.Shape(2, 8, 2, 64, 64, rope_type=0)
    rng = np.random.default_rng(6)
    c, s = O.rope_tables(64, 64, 1e4)
    n, start = 21, 7
    kc1, vc1 = random_cache(O, shp, rng)
    kc2, vc2 = kc1.copy(), vc1.copy()
    q = rng.standard_normal((n, shp.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, shp.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, shp.kv_dim)).astype(np.float32)
    pre = O.attn_prefill(shp, 1, start, n, q.copy(), k.copy(), v, kc1, vc1, c, s)
    for i in range(n):
        d = O.attn_decode(shp, 1, start + i, q[i].copy(), k[i].copy(), v[i].copy(), kc2, vc2, c, s)
        assert np.array_equal(pre[i], d)
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)


@pytest.mark.parametrize("threads", [1, 3, 8, 40])
def test_head_parallel_decode_is_bit_identical(oracle_mod, threads):
    """The CPU baseline's head-parallel variant splits q heads over threads
    without touching a head's arithmetic: outputs and caches equal the
    single-thread oracle bit for bit (thread counts below, at and above the
    head count)."""
    O = oracle_mod
    shp = O.Shape(2, 32, 4, 64, 256, rope_type=0)
    rng = np.random.default_rng(9 + threads)
    c, s = O.rope_tables(256, 64, 1e4)
    kc1, vc1 = random_cache(O, shp, rng)
    kc2, vc2 = kc1.copy(), vc1.copy()
    q = rng.standard_normal(shp.q_dim).astype(np.float32)
    k = rng.standard_normal(shp.kv_dim).astype(np.float32)
    v = rng.standard_normal(shp.kv_dim).astype(np.float32)
    a = O.attn_decode(shp, 1, 200, q.copy(), k.copy(), v, kc1, vc1, c, s)
    b = O.attn_decode_mt(shp, 1, 200, q.copy(), k.copy(), v, kc2, vc2, c, s, threads)
    assert np.array_equal(a, b)
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)


@pytest.mark.parametrize("threads,qkn", [(1, False), (5, False), (16, True), (40, False)])
def test_head_parallel_prefill_is_bit_identical(oracle_mod, threads, qkn):
    """The head-parallel prefill (all prologues first, then each thread's q
    heads over every token) equals the serial oracle bit for bit: outputs and
    caches, with a cached prefix, with and without QK-norm."""
    O = oracle_mod
    shp = O.Shape(2, 16, 4, 64, 128, rope_type=1 if qkn else 0)
    rng = np.random.default_rng(31 + threads)
    c, s = O.rope_tables(128, 64, 1e4)
    start, n = 20, 37
    kc1, vc1 = random_cache(O, shp, rng)
    kc2, vc2 = kc1.copy(), vc1.copy()
    q = rng.standard_normal((n, shp.q_dim)).astype(np.float32)
    k = rng.standard_normal((n, shp.kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, shp.kv_dim)).astype(np.float32)
    qn = (rng.standard_normal(64) * 0.5 + 1).astype(np.float32) if qkn else None
    kn = (rng.standard_normal(64) * 0.5 + 1).astype(np.float32) if qkn else None
    a = O.attn_prefill(shp, 1, start, n, q.copy(), k.copy(), v, kc1, vc1, c, s,
                       q_norm=qn, k_norm=kn, eps=1e-6)
    b = O.attn_prefill_mt(shp, 1, start, n, q.copy(), k.copy(), v, kc2, vc2, c, s, threads,
                          q_norm=qn, k_norm=kn, eps=1e-6)
    assert np.array_equal(a, b)
    assert np.array_equal(kc1, kc2) and np.array_equal(vc1, vc2)


def test_out_of_range_is_rejected(oracle_mod):
    O = oracle_mod
    shp = O.Shape(1, 4, 2, 64, 16)
    c, s = O.rope_tables(16, 64, 1e4)
    kc = np.zeros(shp.cache_elems(), np.uint16)
    vc = kc.copy()
    q = np.zeros((4, shp.q_dim), np.float32)
    k = np.zeros((4, shp.kv_dim), np.float32)
    with pytest.raises(ValueError):
        O.attn_prefill(shp, 0, 14, 4, q, k, k.copy(), kc, vc, c, s)
    with pytest.raises(ValueError):
        O.attn_decode(shp, 0, 16, q[0].copy(), k[0].copy(), k[0].copy(), kc, vc, c, s)
