"""Pins the oracle's RoPE tables (model.c:545-556) and rotation (tensor.c:531-603).

Checks: the reference's tables (tests/golden/rope_tables.npz) bit for bit,
closed-form invariants, and, where the reference harness is built, the
reference's rope() on random inputs bit for bit.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN, needs_ref


def test_tables_match_reference_golden(oracle_mod):
    z = np.load(os.path.join(GOLDEN, "rope_tables.npz"))
    for i in range(3):
        S, D, base = z[f"cfg{i}"]
        c, s = oracle_mod.rope_tables(int(S), int(D), float(base))
        assert np.array_equal(c.view(np.uint32), z[f"cos{i}"].view(np.uint32))
        assert np.array_equal(s.view(np.uint32), z[f"sin{i}"].view(np.uint32))


@pytest.mark.parametrize("S,D,base", [(2048, 64, 1e4), (8192, 64, 5e5), (512, 128, 1e4)])
def test_table_invariants(oracle_mod, S, D, base):
    c, s = oracle_mod.rope_tables(S, D, base)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)          # pos 0: no rotation
    assert np.max(np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1)) < 1e-6
    # frequency i = base^(-2i/D): column 0 rotates by exactly pos radians
    pos = np.arange(S, dtype=np.float64)
    assert np.max(np.abs(c[:, 0] - np.cos(pos))) < 2e-6
    # the last column rotates slowest; a textbook double-precision table agrees
    i = np.arange(D // 2)
    theta = pos[:, None] / base ** (2 * i[None, :] / D)
    assert np.max(np.abs(c - np.cos(theta))) < 5e-4 * max(1.0, S / 2048)
    assert np.max(np.abs(s - np.sin(theta))) < 5e-4 * max(1.0, S / 2048)


@pytest.mark.parametrize("rope_type", [0, 1])
def test_rotation_closed_form(oracle_mod, rope_type):
    D, Hq, Hkv = 64, 4, 2
    rng = np.random.default_rng(7)
    c, s = oracle_mod.rope_tables(300, D, 1e4)
    q = rng.standard_normal(Hq * D).astype(np.float32)
    k = rng.standard_normal(Hkv * D).astype(np.float32)
    q0, k0 = q.copy(), k.copy()
    oracle_mod.rope(q, k, D, Hq, Hkv, c[0], s[0], rope_type)
    assert np.array_equal(q, q0) and np.array_equal(k, k0)      # identity at pos 0
    pos = 257
    oracle_mod.rope(q, k, D, Hq, Hkv, c[pos], s[pos], rope_type)
    half = D // 2
    for x0, x in ((q0, q), (k0, k)):
        x0 = x0.reshape(-1, D).astype(np.float64)
        x = x.reshape(-1, D)
        if rope_type == 0:
            a, b = x0[:, 0::2], x0[:, 1::2]
            ra, rb = x[:, 0::2], x[:, 1::2]
        else:
            a, b = x0[:, :half], x0[:, half:]
            ra, rb = x[:, :half], x[:, half:]
        cc, ss = c[pos].astype(np.float64), s[pos].astype(np.float64)
        # two rounded products and one rounded add/sub: within 2 ulp of exact
        exa, exb = a * cc - b * ss, a * ss + b * cc
        assert np.max(np.abs(ra - exa)) < 4e-7 * max(1, np.max(np.abs(exa)))
        assert np.max(np.abs(rb - exb)) < 4e-7 * max(1, np.max(np.abs(exb)))
        # rotations preserve each pair's norm
        assert np.allclose(ra.astype(np.float64) ** 2 + rb ** 2, a ** 2 + b ** 2, rtol=1e-5)


def test_rotation_uses_no_fma(oracle_mod):
    """Picks inputs where a fused multiply-add would differ from two rounded
    operations, so an FMA-contracted build fails this test."""
    rng = np.random.default_rng(11)
    c, s = oracle_mod.rope_tables(64, 64, 1e4)
    for _ in range(50):
        q = rng.standard_normal(64).astype(np.float32)
        k = rng.standard_normal(64).astype(np.float32)
        q1 = q.copy()
        oracle_mod.rope(q1, k.copy(), 64, 1, 1, c[37], s[37], 0)
        a, b = q[0::2], q[1::2]
        want = (a * c[37] - b * s[37]).astype(np.float32)   # numpy float32: separately rounded
        assert np.array_equal(q1[0::2], want)


@needs_ref
@pytest.mark.parametrize("rope_type", [0, 1])
def test_rotation_matches_reference(oracle_mod, rope_type):
    R = oracle_mod.ref()
    rng = np.random.default_rng(5 + rope_type)
    for D, Hq, Hkv in [(64, 32, 4), (128, 8, 8), (32, 4, 2)]:
        c, s = oracle_mod.rope_tables(600, D, 1e4)
        for pos in (1, 255, 599):
            q = (rng.standard_normal(Hq * D) * 3).astype(np.float32)
            k = (rng.standard_normal(Hkv * D) * 3).astype(np.float32)
            q1, k1, q2, k2 = q.copy(), k.copy(), q.copy(), k.copy()
            oracle_mod.rope(q1, k1, D, Hq, Hkv, c[pos], s[pos], rope_type)
            R.rope(q2, k2, D, Hq, Hkv, c[pos].copy(), s[pos].copy(), rope_type)
            assert np.array_equal(q1.view(np.uint32), q2.view(np.uint32))
            assert np.array_equal(k1.view(np.uint32), k2.view(np.uint32))
