"""Attention results the mathematics fixes, checked on the GPU without the
oracle (model.c:848-892 decode, 1054-1089 prefill):

  * the first position attends to itself alone: decode at pos 0 and the first
    prompt token return their own (fp16-rounded) v row, bit for bit;
  * q = 0 makes every score 0, so the weights are equal and each output is the
    mean of the V rows up to its position (decode: rows 0..pos; prefill: token
    i over rows 0..start+i, which also pins the causal limit of every token);
  * V rows that are constant per kv head make every output the constant of
    its head's kv head (head h reads kv head h / (n_heads / n_kv_heads));
  * a prompt token's output does not depend on the later tokens: changing
    their q, k, v leaves the earlier outputs bit-identical.
Values are fp16-representable where a result is compared bit for bit, so the
rounding of the append is exact whatever its tie rule.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def f16_values(rng, shape, scale=1.0):
    """Normal values rounded to fp16 and back: exact under any fp16 rounding."""
    return (rng.standard_normal(shape) * scale).astype(np.float16).astype(np.float32)


def new_cache(gpu, cfg, rows, rng, v_fn=None):
    """Caches with rows 0..rows-1 of fp16 values (every v row of a layer from
    v_fn(layer) when given)."""
    L, S, kv = cfg.n_layers, cfg.max_seq_len, cfg.kv_dim
    kc = np.zeros((L, S, kv), np.float16)
    vc = np.zeros((L, S, kv), np.float16)
    if rows:
        kc[:, :rows] = rng.standard_normal((L, rows, kv)).astype(np.float16)
        if v_fn is None:
            vc[:, :rows] = rng.standard_normal((L, rows, kv)).astype(np.float16)
        else:
            for l in range(L):
                for t in range(rows):
                    vc[l, t] = v_fn(l).astype(np.float16)
    cache = gpu.KVCache(cfg)
    cache.load(kc.view(np.uint16).reshape(-1), vc.view(np.uint16).reshape(-1))
    return cache, kc.astype(np.float32), vc.astype(np.float32)


def run_decode(gpu, cache, cfg, pos, q, k, v):
    L = cfg.n_layers
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(np.ascontiguousarray(x)) for x in (q, k, v))
    dout = gpu.DeviceBuffer(L * cfg.q_dim * 4)
    gpu.decode(cache, 0, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, L)
    gpu.synchronize()
    return dout.download(np.float32, (L, cfg.n_heads, cfg.head_dim))


def run_prefill(gpu, cache, cfg, start, n, q, k, v):
    L = cfg.n_layers
    dq, dk, dv = (gpu.DeviceBuffer.from_numpy(np.ascontiguousarray(x)) for x in (q, k, v))
    dout = gpu.DeviceBuffer(L * n * cfg.q_dim * 4)
    gpu.prefill(cache, 0, start, n, dq.ptr, dk.ptr, dv.ptr, dout.ptr, None, L)
    gpu.synchronize()
    return dout.download(np.float32, (L, n, cfg.n_heads, cfg.head_dim))


DIMS = [(2, 32, 4, 64, 2048, 0), (2, 8, 8, 128, 2048, 1), (2, 12, 2, 64, 2048, 0),
        (1, 32, 8, 64, 2048, 0)]
IDS = ["gqa8_d64", "mha_d128_qwen", "gqa6_d64", "gqa4_d64"]


@pytest.mark.parametrize("dims", DIMS, ids=IDS)
def test_decode_at_pos0_returns_the_new_v_row_exactly(gpu, dims):
    L, Hq, Hkv, D, S, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, 1e4, rt)
    rng = np.random.default_rng(1)
    print(f"[case] closed form: decode pos 0 {dims}", flush=True)
    cache, _, _ = new_cache(gpu, cfg, 0, rng)
    q = rng.standard_normal((L, cfg.q_dim)).astype(np.float32) * 3
    k = rng.standard_normal((L, cfg.kv_dim)).astype(np.float32)
    v = f16_values(rng, (L, cfg.kv_dim))
    out = run_decode(gpu, cache, cfg, 0, q, k, v)
    cache.free()
    G = Hq // Hkv
    expect = v.reshape(L, Hkv, D)[:, np.arange(Hq) // G]
    assert np.array_equal(out, expect)


@pytest.mark.parametrize("pos", [1, 37, 300, 1000, 2047])
@pytest.mark.parametrize("dims", DIMS, ids=IDS)
def test_decode_with_zero_q_averages_the_v_rows(gpu, dims, pos):
    L, Hq, Hkv, D, S, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, 1e4, rt)
    rng = np.random.default_rng(pos)
    print(f"[case] closed form: decode q=0 {dims} pos {pos}", flush=True)
    cache, _, vc = new_cache(gpu, cfg, pos, rng)
    q = np.zeros((L, cfg.q_dim), np.float32)
    k = rng.standard_normal((L, cfg.kv_dim)).astype(np.float32)
    v = f16_values(rng, (L, cfg.kv_dim))
    out = run_decode(gpu, cache, cfg, pos, q, k, v)
    cache.free()
    rows = np.concatenate([vc[:, :pos].astype(np.float64), v[:, None].astype(np.float64)], 1)
    mean = rows.mean(1).reshape(L, Hkv, D)[:, np.arange(Hq) // (Hq // Hkv)]
    err = np.abs(out - mean).max()
    assert err <= 2e-6 * max(1.0, np.abs(rows).max()), err


@pytest.mark.parametrize("pos", [0, 5, 700])
def test_decode_reads_the_kv_head_of_its_group(gpu, pos):
    """V rows of kv head j all equal 2^j * w (w one fp16 row): every output of
    q head h is 2^(h // G) * w, whatever the weights."""
    L, Hq, Hkv, D, S = 2, 32, 8, 64, 1024
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, 1e4, 0)
    rng = np.random.default_rng(7)
    w = f16_values(rng, D)
    vrow = np.concatenate([w * 2.0 ** j for j in range(Hkv)]).astype(np.float32)
    print(f"[case] closed form: GQA mapping pos {pos}", flush=True)
    cache, _, _ = new_cache(gpu, cfg, pos, rng, v_fn=lambda l: vrow)
    q = rng.standard_normal((L, cfg.q_dim)).astype(np.float32) * 2
    k = rng.standard_normal((L, cfg.kv_dim)).astype(np.float32)
    v = np.tile(vrow, (L, 1))
    out = run_decode(gpu, cache, cfg, pos, q, k, v)
    cache.free()
    expect = np.stack([w * 2.0 ** (h // (Hq // Hkv)) for h in range(Hq)])
    for l in range(L):
        err = np.abs(out[l] - expect) / np.maximum(np.abs(expect), 1e-30)
        assert err.max() <= 1e-5, (l, err.max())


@pytest.mark.parametrize("start,n", [(0, 1), (0, 70), (0, 300), (100, 129), (900, 64)])
@pytest.mark.parametrize("dims", DIMS[:3], ids=IDS[:3])
def test_prefill_with_zero_q_averages_each_tokens_rows(gpu, dims, start, n):
    L, Hq, Hkv, D, S, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, 1024, 1e4, rt)
    rng = np.random.default_rng(start + n)
    print(f"[case] closed form: prefill q=0 {dims} start {start} n {n}", flush=True)
    cache, _, vc = new_cache(gpu, cfg, start, rng)
    q = np.zeros((L, n, cfg.q_dim), np.float32)
    k = rng.standard_normal((L, n, cfg.kv_dim)).astype(np.float32)
    v = f16_values(rng, (L, n, cfg.kv_dim))
    out = run_prefill(gpu, cache, cfg, start, n, q, k, v)
    cache.free()
    rows = np.concatenate([vc[:, :start], v], 1).astype(np.float64)   # [L][start+n][kv]
    means = np.cumsum(rows, 1)[:, start:] / np.arange(start + 1, start + n + 1)[None, :, None]
    expect = means.reshape(L, n, Hkv, D)[:, :, np.arange(Hq) // (Hq // Hkv)]
    err = np.abs(out - expect).max()
    assert err <= 2e-6 * max(1.0, np.abs(rows).max()), err
    if start == 0:   # the first token sees only its own row
        own = v[:, 0].reshape(L, Hkv, D)[:, np.arange(Hq) // (Hq // Hkv)]
        assert np.array_equal(out[:, 0], own)


@pytest.mark.parametrize("start,n,i0", [(0, 300, 37), (0, 512, 256), (64, 200, 1), (10, 130, 129)])
@pytest.mark.parametrize("dims", DIMS[:2], ids=IDS[:2])
def test_prefill_outputs_ignore_later_tokens(gpu, dims, start, n, i0):
    """Tokens before i0 get bit-identical outputs when the q, k, v of tokens
    i0.. change (their keys are masked, so their weights are exactly 0)."""
    L, Hq, Hkv, D, S, rt = dims
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, 1024, 1e4, rt)
    rng = np.random.default_rng(n + i0)
    print(f"[case] closed form: prefill causality {dims} start {start} n {n} i0 {i0}", flush=True)
    q = rng.standard_normal((L, n, cfg.q_dim)).astype(np.float32) * 2
    k = rng.standard_normal((L, n, cfg.kv_dim)).astype(np.float32)
    v = rng.standard_normal((L, n, cfg.kv_dim)).astype(np.float32)
    outs = []
    for r in range(2):
        if r == 1:
            q[:, i0:] = rng.standard_normal((L, n - i0, cfg.q_dim)) * 5
            k[:, i0:] = rng.standard_normal((L, n - i0, cfg.kv_dim)) * 5
            v[:, i0:] = rng.standard_normal((L, n - i0, cfg.kv_dim)) * 5
        cache, _, _ = new_cache(gpu, cfg, start, np.random.default_rng(3))
        outs.append(run_prefill(gpu, cache, cfg, start, n, q, k, v))
        cache.free()
    assert np.array_equal(outs[0][:, :i0], outs[1][:, :i0])
    assert not np.array_equal(outs[0][:, i0:], outs[1][:, i0:])
