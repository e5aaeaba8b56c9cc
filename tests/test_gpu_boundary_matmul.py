"""gpu_try_matmul (gpu_hip.c) on the GPU, driven from C by
tests/c/test_gpu_matmul the way picolm's matmul / matmul_dual call it.

Checks: every uploaded Q4_K / Q6_K / Q8_0 matrix (the seven projections per
layer and the output matrix) returns 0 with outputs bit-identical to the
oracle's matmul (the reference's x86-64 AVX2 vec_dot); F32 / F16 matrices
fall back (-1, nothing written); an unknown pointer, a wrong d or a wrong
type fall back; PICOLM_GPU_LAYERS=1 leaves later layers' matrices on the CPU
(the output matrix stays on the GPU, gpu.c:457-458); PICOLM_HIP_MATMUL=0
uploads nothing.  Head layouts with q_dim = n_heads * head_dim equal to,
twice and half of n_embd (the q projection has q_dim rows)."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from picolm_amd import synth as S

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "c", "test_gpu_matmul")
Q8, Q4K, Q6K, F32, F16 = 8, 12, 14, 0, 1


def run(tmp_path, O, dims, types, type_out, seed, env_extra=None):
    L, n_embd, n_ffn, n_heads, n_kv, hd, vocab = dims
    rng = np.random.default_rng(seed)
    kv_dim, q_dim = n_kv * hd, n_heads * hd
    shapes = [(q_dim, n_embd), (kv_dim, n_embd), (kv_dim, n_embd), (n_embd, q_dim),
              (n_ffn, n_embd), (n_ffn, n_embd), (n_embd, n_ffn)]
    mats = []
    for l in range(L):
        for i, (d, n) in enumerate(shapes):
            mats.append((types[l][i], n, d))
    mats.append((type_out, n_embd, vocab))
    data = []
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        np.array(dims, np.int32).tofile(f)
        np.array([t for row in types for t in row] + [type_out], np.int32).tofile(f)
        for qt, n, d in mats:
            W = S.random_weights(rng, qt, n, d)
            x = rng.standard_normal(n).astype(np.float32)
            W.tofile(f)
            x.tofile(f)
            data.append((W, x))
    env = dict(os.environ)
    env["PICOLM_HIP_GEMV_EXACT"] = "1"   # bit-exact order unless a test asks otherwise
    env.update(env_extra or {})
    print(f"[case] matmul dims {dims} types {types} out {type_out} env {env_extra}", flush=True)
    r = subprocess.run([EXE, str(fin), str(fout)], env=env, capture_output=True, text=True,
                       timeout=240)
    assert r.returncode == 0, r.stderr
    buf = open(fout, "rb").read()
    off = 0

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(buf, dtype=dtype, count=count, offset=off)
        off += a.nbytes
        return a
    rc_init, rc_up = take(np.int32, 2)
    res = []
    for qt, n, d in mats:
        rc = int(take(np.int32, 1)[0])
        res.append((rc, take(np.float32, d)))
    neg = take(np.int32, 3)
    return (rc_init, rc_up), mats, data, res, neg


DIMS = (2, 512, 1024, 8, 2, 64, 1000)   # L, n_embd, n_ffn, heads, kv heads, head_dim, vocab
TYPES = [[Q4K, Q6K, Q8, Q4K, Q4K, Q8, Q6K],
         [Q6K, Q4K, F32, Q8, F16, Q4K, Q4K]]


# q_dim = n_heads * head_dim differs from n_embd: Qwen3-style (q_dim 2 n_embd)
# and the other way round; the q and o projections are d x n and n x d
QDIMS = [DIMS, (2, 256, 512, 4, 2, 128, 700), (2, 512, 512, 2, 1, 128, 300)]


@pytest.mark.parametrize("dims", QDIMS, ids=["q=e", "q=2e", "q=e/2"])
def test_matmul_offload_bit_exact(tmp_path, oracle_mod, dims):
    O = oracle_mod
    rcs, mats, data, res, neg = run(tmp_path, O, dims, TYPES, Q6K, seed=1)
    assert rcs == (0, 0)
    for (qt, n, d), (W, x), (rc, out) in zip(mats, data, res):
        if qt in (F32, F16):
            assert rc == -1 and not out.any()
            continue
        assert rc == 0, (qt, n, d)
        want = O.matmul(W, x, n, d, qt)
        assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), (qt, n, d)
    assert list(neg) == [-1, -1, -1]


def test_matmul_offload_fast_order(tmp_path, oracle_mod):
    """The default GEMV order through gpu_try_matmul: every output within 64
    fp32 ulps of sum |w x| of the float64 dequantize-then-dot."""
    from test_gpu_gemv import assert_fast_close, decode64
    rcs, mats, data, res, neg = run(tmp_path, oracle_mod, DIMS, TYPES, Q6K, seed=4,
                                    env_extra={"PICOLM_HIP_GEMV_EXACT": "0"})
    assert rcs == (0, 0)
    for (qt, n, d), (W, x), (rc, out) in zip(mats, data, res):
        if qt in (F32, F16):
            assert rc == -1 and not out.any()
            continue
        assert rc == 0, (qt, n, d)
        assert_fast_close(out, decode64(qt, W, n, d), x, (qt, n, d))
    assert list(neg) == [-1, -1, -1]


def test_matmul_gpu_layers_limit(tmp_path, oracle_mod):
    O = oracle_mod
    rcs, mats, data, res, _ = run(tmp_path, O, DIMS, TYPES, Q8, seed=2,
                                  env_extra={"PICOLM_GPU_LAYERS": "1"})
    assert rcs == (0, 0)
    for i, ((qt, n, d), (W, x), (rc, out)) in enumerate(zip(mats, data, res)):
        layer = i // 7 if i < 7 * DIMS[0] else None
        if layer == 1 or qt in (F32, F16):
            assert rc == -1 and not out.any()
        else:
            assert rc == 0
            want = O.matmul(W, x, n, d, qt)
            assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


def test_matmul_disabled(tmp_path, oracle_mod):
    rcs, mats, _, res, neg = run(tmp_path, oracle_mod, DIMS, TYPES, Q6K, seed=3,
                                 env_extra={"PICOLM_HIP_MATMUL": "0"})
    assert rcs == (0, 0)
    assert all(rc == -1 and not out.any() for rc, out in res)
    assert list(neg) == [-1, -1, -1]
