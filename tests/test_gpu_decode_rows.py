"""plh_attn_decode_rows, the launch behind the gpu.h decode hook: the same
output and caches as plh_attn_decode / plh_attn_decode_qknorm (model.c:819-892
with 807-817), and the appended rows' fp16 bits (model.c:822-826) also in the
caller's row buffers, device memory or pinned host memory alike."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [
    # (n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, rope_type, layer0,
    #  n_launch_layers, pos, QK-norm)
    (2, 32, 4, 64, 1024, 0, 1, 1, 700, False),   # TinyLlama heads, split launch
    (3, 32, 4, 64, 512, 0, 0, 3, 100, False),    # three layers, one launch, unsplit
    (2, 16, 8, 128, 600, 1, 0, 2, 599, True),    # QWEN rotation + QK-norm, last cache row
    (1, 32, 32, 128, 300, 0, 0, 1, 0, False),    # MHA, position 0
]
IDS = ["tinyllama_split", "three_layers", "qwen_qknorm_last_row", "mha_pos0"]


def host_view(ptr, n):
    return np.ctypeslib.as_array((C.c_uint16 * n).from_address(ptr))


@pytest.mark.parametrize("host_rows", [False, True], ids=["device_rows", "pinned_host_rows"])
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_decode_rows_match_plain_decode(gpu, case, host_rows):
    L, Hq, Hkv, D, S, rt, layer0, nl, pos, qkn = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, 1e4, rt)
    rng = np.random.default_rng(pos + 7 * nl + D)
    print(f"[case] decode_rows {case} host_rows={host_rows}", flush=True)
    kc = np.zeros((L, S, cfg.kv_dim), np.float16)
    vc = np.zeros((L, S, cfg.kv_dim), np.float16)
    kc[:, :pos] = rng.standard_normal((L, pos, cfg.kv_dim))
    vc[:, :pos] = rng.standard_normal((L, pos, cfg.kv_dim))
    q = (rng.standard_normal((nl, cfg.q_dim)) * 2).astype(np.float32)
    k = rng.standard_normal((nl, cfg.kv_dim)).astype(np.float32)
    v = rng.standard_normal((nl, cfg.kv_dim)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal((2, nl, D))).astype(np.float32)
    nrow = nl * cfg.kv_dim

    results = {}
    for mode in ("plain", "rows"):
        cache = gpu.KVCache(cfg)
        cache.load(kc.view(np.uint16).reshape(-1), vc.view(np.uint16).reshape(-1))
        dq, dk, dv = (gpu.DeviceBuffer.from_numpy(x) for x in (q, k, v))
        dqn, dkn = (gpu.DeviceBuffer.from_numpy(x) for x in nw)
        dout = gpu.DeviceBuffer(nl * cfg.q_dim * 4)
        norms = dict(q_norm=dqn.ptr, k_norm=dkn.ptr, norm_eps=1e-6) if qkn else {}
        rows = None
        if mode == "plain":
            gpu.decode(cache, layer0, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, nl, **norms)
            gpu.synchronize()
        else:
            if host_rows:
                kr, vr = gpu.lib.plh_host_alloc(nrow * 2), gpu.lib.plh_host_alloc(nrow * 2)
                assert kr and vr
                host_view(kr, nrow)[:] = 0xFFFF
                host_view(vr, nrow)[:] = 0xFFFF
            else:
                bk, bv = gpu.DeviceBuffer(nrow * 2), gpu.DeviceBuffer(nrow * 2)
                kr, vr = bk.ptr, bv.ptr
            gpu.decode_rows(cache, layer0, pos, dq.ptr, dk.ptr, dv.ptr, dout.ptr, kr, vr, nl,
                            **norms)
            gpu.synchronize()
            if host_rows:
                rows = (host_view(kr, nrow).copy(), host_view(vr, nrow).copy())
                gpu.check(gpu.lib.plh_host_free(kr), "plh_host_free")
                gpu.check(gpu.lib.plh_host_free(vr), "plh_host_free")
            else:
                rows = (bk.download(np.uint16, (nrow,)), bv.download(np.uint16, (nrow,)))
                bk.free()
                bv.free()
        out = dout.download(np.float32, (nl, cfg.q_dim))
        gk, gv = cache.fetch()
        results[mode] = (out, gk.reshape(L, S, cfg.kv_dim), gv.reshape(L, S, cfg.kv_dim), rows)
        for b in (dq, dk, dv, dqn, dkn, dout):
            b.free()
        cache.free()

    out0, gk0, gv0, _ = results["plain"]
    out1, gk1, gv1, (kr, vr) = results["rows"]
    assert np.array_equal(out0, out1)
    assert np.array_equal(gk0, gk1) and np.array_equal(gv0, gv1)
    for li in range(nl):
        sl = slice(li * cfg.kv_dim, (li + 1) * cfg.kv_dim)
        assert np.array_equal(kr[sl], gk1[layer0 + li, pos])
        assert np.array_equal(vr[sl], gv1[layer0 + li, pos])
    # the appended rows are the only change to the caches
    kc_bits, vc_bits = kc.view(np.uint16), vc.view(np.uint16)
    mask = np.ones((L, S), bool)
    mask[layer0:layer0 + nl, pos] = False
    assert np.array_equal(gk1[mask], kc_bits[mask]) and np.array_equal(gv1[mask], vc_bits[mask])


def test_decode_rows_rejects_null_row_buffers(gpu):
    cfg = gpu.AttnConfig(1, 8, 2, 64, 64, 1e4, 0)
    cache = gpu.KVCache(cfg)
    dq = gpu.DeviceBuffer(cfg.q_dim * 4)
    dkv = gpu.DeviceBuffer(cfg.kv_dim * 4)
    dout = gpu.DeviceBuffer(cfg.q_dim * 4)
    rows = gpu.DeviceBuffer(cfg.kv_dim * 2)
    with pytest.raises(gpu.PicolmHipError):
        gpu.decode_rows(cache, 0, 3, dq.ptr, dkv.ptr, dkv.ptr, dout.ptr, rows.ptr, None)
    for b in (dq, dkv, dout, rows):
        b.free()
    cache.free()
