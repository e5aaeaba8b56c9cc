"""Weight GEMV on the GPU (plh_gemv, the gpu_try_matmul path) against the
oracle.  The exact order (plh_set_tuning key 10 = 1), bit for bit: every
output of every row equals the reference's vec_dot in its x86-64 AVX2 build
(the oracle is pinned to it in tests/test_oracle_gemv.py).  The default fast
order (x as fixed-point int8 digits, integer dot products): every output
within 64 fp32 ulps of sum |w x| of the float64 dequantize-then-dot, the
bound the oracle's own AVX2 order meets (tests/test_oracle_gemv.py), for
plain, tiny, large and outlier-heavy x.

Shapes: the TinyLlama projections (q/o 2048x2048, k/v 256x2048, gate/up
5632x2048, down 2048x5632), a Llama-2 MLP row length (11008) whose term
buffer limits a workgroup's rows, row counts that leave partial workgroups,
and a vocabulary-sized output projection."""
import numpy as np
import pytest

import picolm_amd as P
from picolm_amd import gemv as G
from picolm_amd import synth as S

pytestmark = pytest.mark.gpu


@pytest.fixture
def exact_order(gpu):
    """The bit-exact GEMV order for one test."""
    gpu.check(gpu.lib.plh_set_tuning(10, 1), "plh_set_tuning")
    yield
    gpu.check(gpu.lib.plh_set_tuning(10, 0), "plh_set_tuning")


def decode64(qtype, W, n, d):
    from test_oracle_gemv import _decode64
    name = {G.TYPE_Q4_K: "q4_K", G.TYPE_Q6_K: "q6_K", G.TYPE_Q8_0: "q8_0"}[qtype]
    return _decode64(name, W, n, d)


def assert_fast_close(got, W64, x, what):
    """|got - float64 dot| <= 64 ulps of sum |w x| (the AVX2 order's bound)."""
    x64 = x.astype(np.float64)
    exact = W64 @ x64
    bound = 64 * np.finfo(np.float32).eps * (np.abs(W64) @ np.abs(x64)) + 1e-30
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= bound), (what, float(np.max(err / bound)))
    return float(np.max(err / bound))

SHAPES = [  # (qtype, n, d)
    (G.TYPE_Q4_K, 2048, 2048), (G.TYPE_Q4_K, 2048, 256), (G.TYPE_Q4_K, 2048, 5632),
    (G.TYPE_Q4_K, 5632, 2048), (G.TYPE_Q4_K, 256, 77), (G.TYPE_Q4_K, 11008, 129),
    (G.TYPE_Q6_K, 2048, 2048), (G.TYPE_Q6_K, 5632, 2048), (G.TYPE_Q6_K, 2048, 32000),
    (G.TYPE_Q6_K, 256, 3), (G.TYPE_Q6_K, 11008, 65),
    (G.TYPE_Q8_0, 2048, 2048), (G.TYPE_Q8_0, 5632, 2048), (G.TYPE_Q8_0, 32, 5),
    (G.TYPE_Q8_0, 96, 1000), (G.TYPE_Q8_0, 11008, 100),
]


@pytest.mark.parametrize("qtype,n,d", SHAPES)
def test_gemv_bit_exact(gpu, oracle_mod, exact_order, qtype, n, d):
    O = oracle_mod
    rng = np.random.default_rng(n * 7 + d + qtype)
    print(f"[case] gemv type {qtype} n {n} d {d}", flush=True)
    W = S.random_weights(rng, qtype, n, d)
    Wd = G.QMatrix(qtype, n, d, W)
    for trial, xs in enumerate((1.0, 1e-3, 40.0)):
        x = (rng.standard_normal(n) * xs).astype(np.float32)
        dx = P.DeviceBuffer.from_numpy(x)
        dout = P.DeviceBuffer(d * 4)
        G.matmul(dout.ptr, dx.ptr, Wd)
        got = dout.download(np.float32, (d,))
        want = O.matmul(W, x, n, d, qtype)
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, (trial, bad[:8], got[bad[:4]], want[bad[:4]])
        dx.free()
        dout.free()
    Wd.free()


@pytest.mark.parametrize("qtype,n,d", SHAPES)
def test_gemv_fast_order(gpu, qtype, n, d):
    rng = np.random.default_rng(n * 7 + d + qtype)
    print(f"[case] fast gemv type {qtype} n {n} d {d}", flush=True)
    W = S.random_weights(rng, qtype, n, d)
    W64 = decode64(qtype, W, n, d)
    Wd = G.QMatrix(qtype, n, d, W)
    worst = 0.0
    for trial, xs in enumerate((1.0, 1e-3, 40.0, "outliers")):
        if xs == "outliers":
            # one element in every 32-element block 300x the rest, and blocks
            # of zeros and of tiny values
            x = rng.standard_normal(n).astype(np.float32)
            x[rng.integers(0, 32) + 32 * np.arange(n // 32)] *= 300.0
            x[: n // 4] = 0.0
            x[n // 4: n // 2] *= 1e-30
        else:
            x = (rng.standard_normal(n) * xs).astype(np.float32)
        dx = P.DeviceBuffer.from_numpy(x)
        dout = P.DeviceBuffer(d * 4)
        G.matmul(dout.ptr, dx.ptr, Wd)
        got = dout.download(np.float32, (d,))
        worst = max(worst, assert_fast_close(got, W64, x, (qtype, n, d, trial)))
        dx.free()
        dout.free()
    print(f"[fast] type {qtype} n {n} d {d}: worst error / bound {worst:.3f}")
    Wd.free()


@pytest.mark.parametrize("order", ["exact", "fast"])
def test_gemv_repeat_and_special_blocks(gpu, oracle_mod, order):
    """Zero scales, all-zero x and repeated calls (no state between calls):
    bit-exact in the exact order, within the bound in the fast one."""
    gpu.check(gpu.lib.plh_set_tuning(10, 1 if order == "exact" else 0), "plh_set_tuning")
    try:
        _repeat_and_special_blocks(gpu, oracle_mod, order == "exact")
    finally:
        gpu.check(gpu.lib.plh_set_tuning(10, 0), "plh_set_tuning")


def _repeat_and_special_blocks(gpu, oracle_mod, exact):
    O = oracle_mod
    rng = np.random.default_rng(5)
    n, d = 512, 64
    for qtype in (G.TYPE_Q4_K, G.TYPE_Q6_K, G.TYPE_Q8_0):
        W = S.random_weights(rng, qtype, n, d)
        rb = G.row_bytes(qtype, n)
        blocks = W.reshape(d, -1, G.BLOCK[qtype][1])
        if qtype == G.TYPE_Q4_K:
            blocks[::3, :, 0:4] = 0          # d = dmin = 0 on every third row
        elif qtype == G.TYPE_Q6_K:
            blocks[::3, :, 208:210] = 0
        else:
            blocks[::3, :, 0:2] = 0
        assert W.shape == (d, rb)
        Wd = G.QMatrix(qtype, n, d, W)
        for x in (np.zeros(n, np.float32), rng.standard_normal(n).astype(np.float32)):
            dx = P.DeviceBuffer.from_numpy(x)
            dout = P.DeviceBuffer(d * 4)
            want = O.matmul(W, x, n, d, qtype)
            for _ in range(2):
                G.matmul(dout.ptr, dx.ptr, Wd)
                got = dout.download(np.float32, (d,))
                if exact:
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
                else:
                    assert_fast_close(got, decode64(qtype, W, n, d), x, qtype)
            assert not got[::3].any()
            dx.free()
            dout.free()
        Wd.free()


def test_gemv_rejects_bad_calls(gpu):
    assert P.lib.plh_gemv(2, 32, 4, None, None, None) != 0           # Q4_0: no kernel
    buf = P.DeviceBuffer(1024)
    assert P.lib.plh_gemv(G.TYPE_Q4_K, 100, 4, buf.ptr, buf.ptr, buf.ptr) != 0
    assert P.lib.plh_gemv(G.TYPE_Q8_0, 32, 1, None, buf.ptr, buf.ptr) != 0
    buf.free()


@pytest.mark.parametrize("qtype,n,d,nb", [
    (G.TYPE_Q4_K, 2048, 2048, 13), (G.TYPE_Q6_K, 5632, 2048, 9),
    (G.TYPE_Q8_0, 2048, 256, 17), (G.TYPE_Q6_K, 2048, 256, 8),
    (G.TYPE_Q4_K, 2048, 5632, 3)])
def test_matmul_batch_bit_exact(gpu, oracle_mod, qtype, n, d, nb):
    """tensor.c:322-366 matmul_batch: every (row, token) equals the oracle's
    single-vector matmul bit for bit, for token counts around the tile."""
    import ctypes as C
    P, O = gpu, oracle_mod
    rng = np.random.default_rng(qtype * 7 + nb)
    W = S.random_weights(rng, qtype, n, d, S.unit_scale_exp(qtype, n))
    X = rng.standard_normal((nb, n)).astype(np.float32)
    M = G.QMatrix(qtype, n, d, W)
    dx = P.DeviceBuffer.from_numpy(X)
    out = P.DeviceBuffer(4 * nb * d)
    P.check(P.lib.plh_matmul_batch(qtype, n, d, C.c_void_p(M.ptr), C.c_void_p(dx.ptr), nb,
                                   C.c_void_p(out.ptr)), "plh_matmul_batch")
    got = out.download(np.float32, (nb, d))
    for b in range(nb):
        want = O.matmul(W, X[b], n, d, qtype)
        assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), b


@pytest.mark.parametrize("rb", [1, 2, 4, 8])
def test_gemv_fast_order_rows_per_thread(gpu, rb):
    """Every rows-per-thread variant of the fast order (tuning key 3), as a
    single GEMV with the rmsnorm prologue and as a gate/up pair (whose second
    rows are issued after the x staging), within the fast order's bound of
    the float64 product; the pair's silu(gate) * up within that bound carried
    through silu and the product."""
    import ctypes as C
    rng = np.random.default_rng(900 + rb)
    qt, n, d = G.TYPE_Q4_K, 2048, 1000
    Wg = S.random_weights(rng, qt, n, d, S.unit_scale_exp(qt, n))
    Wu = S.random_weights(rng, qt, n, d, S.unit_scale_exp(qt, n))
    g64, u64 = decode64(qt, Wg, n, d), decode64(qt, Wu, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, n).astype(np.float32)
    xs = x.astype(np.float64)
    xn = xs / np.sqrt(np.mean(xs * xs) + 1e-5) * nw
    Gd, Ud = G.QMatrix(qt, n, d, Wg), G.QMatrix(qt, n, d, Wu)
    dx, dnw = P.DeviceBuffer.from_numpy(x), P.DeviceBuffer.from_numpy(nw)
    out = P.DeviceBuffer(4 * d)
    vp = C.c_void_p
    eps32 = np.finfo(np.float32).eps
    P.check(P.lib.plh_set_tuning(3, rb), "plh_set_tuning")
    try:
        print(f"[case] fast gemv rows per thread {rb}", flush=True)
        P.check(P.lib.plh_gemv_ex(qt, n, d, vp(Gd.ptr), vp(dx.ptr), vp(out.ptr), vp(dnw.ptr),
                                  C.c_float(1e-5), None, 0, None, None), "plh_gemv_ex")
        got = out.download(np.float32, (d,)).astype(np.float64)
        want = g64 @ xn
        mag = np.abs(g64) @ np.abs(xn)
        assert np.all(np.abs(got - want) <= 128 * eps32 * mag + 1e-30), rb
        P.check(P.lib.plh_gemv_swiglu(qt, n, d, vp(Gd.ptr), vp(Ud.ptr), vp(dx.ptr), vp(out.ptr),
                                      vp(dnw.ptr), C.c_float(1e-5)), "plh_gemv_swiglu")
        got = out.download(np.float32, (d,)).astype(np.float64)
        g, u = g64 @ xn, u64 @ xn
        want = g / (1.0 + np.exp(-g)) * u
        dg = 128 * eps32 * (np.abs(g64) @ np.abs(xn))
        du = 128 * eps32 * (np.abs(u64) @ np.abs(xn))
        # |d silu(g)/dg| <= 1.1; silu's own rounding a few ulps of the result
        tol = 1.1 * dg * np.abs(u) + np.abs(g) * du + 1.1 * dg * du + 8 * eps32 * np.abs(want)
        assert np.all(np.abs(got - want) <= tol + 1e-30), (rb, float(np.max(np.abs(got - want) / (tol + 1e-30))))
    finally:
        P.check(P.lib.plh_set_tuning(3, 0), "plh_set_tuning")
        for b in (Gd, Ud, dx, dnw, out):
            b.free()
