"""Pins the oracle's Qwen3 QK-norm (model.c:807-817 decode, 1029-1037
prefill): per-head RMSNorm of q and k before the rotation.

Checks:
  * orc_rmsnorm equals the reference's rmsnorm (tensor.c:425-492, built for
    x86-64 with AVX2 like any MI355X host's native build) bit for bit, sizes
    with and without a tail;
  * against float64 mathematics, so that a dropped epsilon, a sum in place of
    the mean or a missing weight fails without the reference;
  * decode and prefill with QK-norm replay the reference's forward passes:
    outputs, caches and the logits of the whole chain bit for bit.
"""
import numpy as np
import pytest

from conftest import needs_ref


def test_rmsnorm_matches_float64(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(1)
    for size in (8, 64, 128, 72):
        for scale in (1e-3, 1.0, 50.0):
            x = (rng.standard_normal(size) * scale).astype(np.float32)
            w = (rng.standard_normal(size) * 0.5 + 1).astype(np.float32)
            eps = 1e-6
            got = O.rmsnorm(x, w, eps).astype(np.float64)
            x64 = x.astype(np.float64)
            want = x64 / np.sqrt(np.mean(x64 * x64) + eps) * w.astype(np.float64)
            np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-30)
    # epsilon matters when the row is tiny: all-zero row stays zero, a row of
    # 1e-4 is pulled well below unit size by eps = 1e-5
    z = O.rmsnorm(np.zeros(64, np.float32), np.ones(64, np.float32), 1e-5)
    assert not z.any()
    t = O.rmsnorm(np.full(64, 1e-4, np.float32), np.ones(64, np.float32), 1e-5)
    assert np.allclose(t, 1e-4 / np.sqrt(1e-8 + 1e-5), rtol=1e-6)


@needs_ref
def test_rmsnorm_matches_reference_bits(oracle_mod):
    O = oracle_mod
    R = O.ref()
    rng = np.random.default_rng(2)
    for size in (8, 16, 64, 128, 72, 13):
        for trial in range(200):
            scale = 10.0 ** rng.uniform(-4, 3)
            x = (rng.standard_normal(size) * scale).astype(np.float32)
            w = rng.standard_normal(size).astype(np.float32)
            eps = float(rng.choice([1e-5, 1e-6, 1e-7]))
            want = np.empty(size, np.float32)
            R.ref_rmsnorm(want, x, w, size, eps)
            got = O.rmsnorm(x, w, eps)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (size, trial)


@needs_ref
@pytest.mark.parametrize("L,Hq,Hkv,D,S,base,rt", [
    (2, 16, 2, 128, 20, 1e6, 1),     # Qwen3 layout: QWEN rotation, D=128, GQA 8
    (1, 8, 2, 64, 24, 1e4, 0),       # LLaMA rotation with QK-norm
])
def test_decode_qknorm_matches_reference_live(oracle_mod, L, Hq, Hkv, D, S, base, rt):
    O = oracle_mod
    shp = O.Shape(L, Hq, Hkv, D, S, base, rt)
    rm = O.RefModel(shp, 0, seed=7)
    R = O.ref()
    rng = np.random.default_rng(8)
    eps = 1e-6
    qw = (rng.standard_normal((L, D)) * 0.5 + 1).astype(np.float32)
    kw = (rng.standard_normal((L, D)) * 0.5 + 1).astype(np.float32)
    for l in range(L):
        R.ref_set_qk_norm(rm.h, l, qw[l], kw[l], eps)
    c, s = O.rope_tables(S, D, base)
    kc = np.zeros(shp.cache_elems(), np.uint16)
    vc = kc.copy()
    try:
        for pos in range(S):
            qs = (rng.standard_normal((L, shp.q_dim)) * 3).astype(np.float32)
            ks = (rng.standard_normal((L, shp.kv_dim)) * 3).astype(np.float32)
            vs = rng.standard_normal((L, shp.kv_dim)).astype(np.float32)
            for l in range(L):
                R.ref_set_decode_qkv(rm.h, l, qs[l], ks[l], vs[l])
            want = np.empty(shp.q_dim, np.float32)
            R.ref_decode(rm.h, pos, L, want)
            for l in range(L):
                out = O.attn_decode(shp, l, pos, qs[l].copy(), ks[l].copy(), vs[l], kc, vc, c, s,
                                    q_norm=qw[l], k_norm=kw[l], eps=eps)
            assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), pos
        assert np.array_equal(kc, rm.kc) and np.array_equal(vc, rm.vc)
    finally:
        rm.close()


@needs_ref
@pytest.mark.parametrize("L,Hq,Hkv,D,S,base,rt,chunks", [
    (2, 16, 2, 128, 48, 1e6, 1, (20, 9)),
    (2, 8, 4, 64, 40, 1e4, 0, (17,)),
])
def test_prefill_qknorm_matches_reference_live(oracle_mod, L, Hq, Hkv, D, S, base, rt, chunks):
    O = oracle_mod
    R = O.ref()
    shp = O.Shape(L, Hq, Hkv, D, S, base, rt)
    rm = O.RefModel(shp, 1, seed=11, w_scale=0.3)
    rng = np.random.default_rng(12)
    eps = 1e-6
    qw = (rng.standard_normal((L, D)) * 0.5 + 1).astype(np.float32)
    kw = (rng.standard_normal((L, D)) * 0.5 + 1).astype(np.float32)
    for l in range(L):
        R.ref_set_qk_norm(rm.h, l, qw[l], kw[l], eps)
    c, s = O.rope_tables(S, D, base)
    kc = np.zeros(shp.cache_elems(), np.uint16)
    vc = kc.copy()
    start = 0
    try:
        for n in chunks:
            toks = rng.integers(0, shp.q_dim, n).astype(np.int32)
            logits = np.empty(shp.q_dim, np.float32)
            R.ref_prefill(rm.h, toks, n, start, logits)
            x = np.empty((n, shp.q_dim), np.float32)
            R.ref_embed(rm.h, toks, n, x.reshape(-1))
            for l in range(L):
                q = np.empty((n, shp.q_dim), np.float32)
                k = np.empty((n, shp.kv_dim), np.float32)
                v = np.empty((n, shp.kv_dim), np.float32)
                R.ref_layer_inputs(rm.h, l, x.reshape(-1), n, q.reshape(-1), k.reshape(-1),
                                   v.reshape(-1))
                a = O.attn_prefill(shp, l, start, n, q, k, v, kc, vc, c, s,
                                   q_norm=qw[l], k_norm=kw[l], eps=eps)
                x = (x + a) + np.float32(0)
            expect = np.empty(shp.q_dim, np.float32)
            R.ref_final_norm(rm.h, np.ascontiguousarray(x[-1]), expect)
            assert np.array_equal(expect.view(np.uint32), logits.view(np.uint32))
            start += n
        assert np.array_equal(kc, rm.kc) and np.array_equal(vc, rm.vc)
    finally:
        rm.close()


def test_qknorm_needs_both_weights(oracle_mod):
    O = oracle_mod
    shp = O.Shape(1, 4, 2, 64, 16)
    c, s = O.rope_tables(16, 64, 1e4)
    kc = np.zeros(shp.cache_elems(), np.uint16)
    vc = kc.copy()
    q = np.ones(shp.q_dim, np.float32)
    k = np.ones(shp.kv_dim, np.float32)
    with pytest.raises(ValueError):
        O.attn_decode(shp, 0, 3, q, k, k.copy(), kc, vc, c, s, q_norm=np.ones(64), k_norm=None)
