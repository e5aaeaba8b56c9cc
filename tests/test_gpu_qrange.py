"""q beyond the fp16 range, on the GPU, against the oracle.

The kernels split q into fp16 hi + lo parts for the MFMA; a q head with an
element at or above 65504 would overflow that split.  Each such head is
scaled by a power of two before the split and the factor moves into its
score scale, which is exact, so the reference's fp32 results (which stay
finite) are matched.  The caches hold small keys (N(0,1) * 2^-12) so that the
scores of |q| ~ 1e5 stay O(1) and the softmax is not one-hot: every term of
the attention matters.  A second case uses |q| ~ 1e30 (one-hot softmax).
Heads with ordinary q are unchanged by the scaling (bit-identical path)."""
import numpy as np
import pytest

from attn_check import assert_attn_close, normal_f32

pytestmark = pytest.mark.gpu

K_SCALE = 2.0 ** -12


def big_q(rng, shape, D, scale):
    """N(0,1) * scale, plus one element of +-4*scale per head (at or above
    65504 for scale >= 16376), and the first head of every row left N(0,1)."""
    q = normal_f32(rng, shape, scale).reshape(-1, D)
    q[np.arange(q.shape[0]), rng.integers(0, D, q.shape[0])] = np.float32(4 * scale)
    q = q.reshape(shape)
    q.reshape(-1, shape[-1])[:, :D] = normal_f32(rng, (int(np.prod(shape[:-1])), D))
    return q


@pytest.mark.parametrize("scale", [3e4, 1e30], ids=["q3e4", "q1e30"])
@pytest.mark.parametrize("dims", [(2, 32, 4, 64, 640, 0), (2, 8, 8, 128, 320, 1)],
                         ids=["gqa8_d64", "mha_d128_qwen"])
def test_decode_large_q(gpu, oracle_mod, dims, scale):
    O = oracle_mod
    L, Hq, Hkv, D, S, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, 1e4, rt)
    rng = np.random.default_rng(int(scale) % 1000 + D)
    pos = S - 3
    kc = np.zeros((L, S, cfg.kv_dim), np.uint16)
    vc = np.zeros((L, S, cfg.kv_dim), np.uint16)
    kc[:, :pos] = O.f32_to_f16(normal_f32(rng, (L, pos, cfg.kv_dim), K_SCALE))
    vc[:, :pos] = O.f32_to_f16(normal_f32(rng, (L, pos, cfg.kv_dim)))
    kc, vc = kc.reshape(-1), vc.reshape(-1)
    q = big_q(rng, (L, cfg.q_dim), D, scale)
    k = normal_f32(rng, (L, cfg.kv_dim), K_SCALE)
    v = normal_f32(rng, (L, cfg.kv_dim))
    print(f"[case] decode large q {dims} scale {scale:g} pos {pos}", flush=True)
    cache = gpu.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = gpu.DeviceBuffer(L * cfg.q_dim * 4)
    gpu.decode(cache, 0, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, L)
    gpu.synchronize()
    out = dout.download(np.float32, (L, cfg.q_dim))
    gk, gv = cache.fetch()
    shp = O.Shape(L, Hq, Hkv, D, S, 1e4, rt)
    cos_t, sin_t = O.rope_tables(S, D, 1e4)
    for l in range(L):
        ref = O.attn_decode(shp, l, pos, q[l].copy(), k[l].copy(), v[l], kc, vc, cos_t, sin_t)
        assert np.all(np.isfinite(ref))
        assert_attn_close(out[l], ref, D, 1e-3, f"layer {l}")
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)


@pytest.mark.parametrize("scale", [3e4, 1e30], ids=["q3e4", "q1e30"])
@pytest.mark.parametrize("dims", [(1, 32, 4, 64, 256, 0), (1, 8, 8, 128, 256, 1)],
                         ids=["gqa8_d64", "mha_d128_qwen"])
def test_prefill_large_q(gpu, oracle_mod, dims, scale):
    O = oracle_mod
    L, Hq, Hkv, D, S, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, 1e4, rt)
    rng = np.random.default_rng(int(scale) % 997 + D)
    start, n = 37, 150
    kc = np.zeros((L, S, cfg.kv_dim), np.uint16)
    vc = np.zeros((L, S, cfg.kv_dim), np.uint16)
    kc[:, :start] = O.f32_to_f16(normal_f32(rng, (L, start, cfg.kv_dim), K_SCALE))
    vc[:, :start] = O.f32_to_f16(normal_f32(rng, (L, start, cfg.kv_dim)))
    kc, vc = kc.reshape(-1), vc.reshape(-1)
    q = big_q(rng, (L, n, cfg.q_dim), D, scale)
    k = normal_f32(rng, (L, n, cfg.kv_dim), K_SCALE)
    v = normal_f32(rng, (L, n, cfg.kv_dim))
    print(f"[case] prefill large q {dims} scale {scale:g} start {start} n {n}", flush=True)
    cache = gpu.KVCache(cfg)
    cache.load(kc, vc)
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v))
    dout = gpu.DeviceBuffer(L * n * cfg.q_dim * 4)
    gpu.prefill(cache, 0, start, n, dq.ptr, dk.ptr, dv.ptr, dout.ptr, None, L)
    gpu.synchronize()
    out = dout.download(np.float32, (L, n, cfg.q_dim))
    gk, gv = cache.fetch()
    shp = O.Shape(L, Hq, Hkv, D, S, 1e4, rt)
    cos_t, sin_t = O.rope_tables(S, D, 1e4)
    rk, rv = kc.copy(), vc.copy()
    for l in range(L):
        ref = O.attn_prefill(shp, l, start, n, q[l].copy(), k[l].copy(), v[l], rk, rv, cos_t,
                             sin_t)
        assert np.all(np.isfinite(ref))
        assert_attn_close(out[l], ref, D, 1e-3, f"layer {l}")
    assert np.array_equal(gk, rk) and np.array_equal(gv, rv)
