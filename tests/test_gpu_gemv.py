"""Weight GEMV on the GPU (plh_gemv, the gpu_try_matmul path) against the
oracle, bit for bit: every output of every row equals the reference's
vec_dot in its x86-64 AVX2 build (the oracle is pinned to it in
tests/test_oracle_gemv.py).

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

SHAPES = [  # (qtype, n, d)
    (G.TYPE_Q4_K, 2048, 2048), (G.TYPE_Q4_K, 2048, 256), (G.TYPE_Q4_K, 2048, 5632),
    (G.TYPE_Q4_K, 5632, 2048), (G.TYPE_Q4_K, 256, 77), (G.TYPE_Q4_K, 11008, 129),
    (G.TYPE_Q6_K, 2048, 2048), (G.TYPE_Q6_K, 5632, 2048), (G.TYPE_Q6_K, 2048, 32000),
    (G.TYPE_Q6_K, 256, 3), (G.TYPE_Q6_K, 11008, 65),
    (G.TYPE_Q8_0, 2048, 2048), (G.TYPE_Q8_0, 5632, 2048), (G.TYPE_Q8_0, 32, 5),
    (G.TYPE_Q8_0, 96, 1000), (G.TYPE_Q8_0, 11008, 100),
]


@pytest.mark.parametrize("qtype,n,d", SHAPES)
def test_gemv_bit_exact(gpu, oracle_mod, qtype, n, d):
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


def test_gemv_repeat_and_special_blocks(gpu, oracle_mod):
    """Zero scales, all-zero x and repeated calls (no state between calls)."""
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
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
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
