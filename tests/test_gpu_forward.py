"""The device forward pass (plh_forward, picolm's model_forward) and its new
pieces against the oracle, on the GPU.

Bit-exact: rmsnorm (every size class: vector part, tail, odd lengths,
in-place), embedding dequantisation of every supported type, the GEMV
epilogues (bias, zero bias, residual) in the exact GEMV order, and, in that
order, the layer-0 KV rows of every forward step (embedding -> rmsnorm ->
GEMV -> RoPE -> fp16 involve no transcendental).  Within tolerance (the
device's expf in silu and the split-K exp2 softmax differ from glibc's expf
in the last bits; the default fast GEMV order sums differently): silu * up
per element, the fast order's epilogues, and the logits / final residual /
KV rows of whole forward passes over LLaMA- and Qwen-shaped models, with
the greedy token checked where the oracle's top two logits are apart.
"""
import contextlib
import ctypes as C

import numpy as np
import pytest

from attn_check import FWD_TOL, FWD_TOL_FAST, KV_TOL, KV_TOL_FAST
from picolm_amd import synth as S

pytestmark = pytest.mark.gpu

Q4K, Q6K, Q8, Q40, F32, F16 = (S.TYPE_Q4_K, S.TYPE_Q6_K, S.TYPE_Q8_0, S.TYPE_Q4_0,
                               S.TYPE_F32, S.TYPE_F16)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@contextlib.contextmanager
def gemv_order(P, order):
    """The GEMV summation order ("exact" or "fast") for a block."""
    P.check(P.lib.plh_set_tuning(10, 1 if order == "exact" else 0), "plh_set_tuning")
    try:
        yield
    finally:
        P.check(P.lib.plh_set_tuning(10, 0), "plh_set_tuning")


@pytest.mark.parametrize("n", [1, 7, 8, 64, 100, 2048, 2051, 5632, 12288])
def test_rmsnorm_bit_exact(gpu, oracle_mod, n):
    P, O = gpu, oracle_mod
    rng = np.random.default_rng(n)
    for scale, eps in ((1.0, 1e-5), (1e-3, 1e-6), (300.0, 1e-5)):
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        dx, dw, do = P.DeviceBuffer.from_numpy(x), P.DeviceBuffer.from_numpy(w), P.DeviceBuffer(4 * n)
        P.check(P.lib.plh_rmsnorm(dx.ptr, dw.ptr, do.ptr, n, C.c_float(eps)), "plh_rmsnorm")
        want = O.rmsnorm(x, w, eps)
        assert np.array_equal(bits(do.download(np.float32, (n,))), bits(want)), (n, scale)
        # in place
        P.check(P.lib.plh_rmsnorm(dx.ptr, dw.ptr, dx.ptr, n, C.c_float(eps)), "plh_rmsnorm")
        assert np.array_equal(bits(dx.download(np.float32, (n,))), bits(want))


def test_rmsnorm_rejects_oversize(gpu):
    P = gpu
    b = P.DeviceBuffer(4 * 16)
    assert P.lib.plh_rmsnorm(b.ptr, b.ptr, b.ptr, 12289, C.c_float(1e-5)) == -1
    assert P.lib.plh_rmsnorm(b.ptr, b.ptr, b.ptr, 0, C.c_float(1e-5)) == -1


@pytest.mark.parametrize("qtype", [F32, F16, Q40, Q8, Q4K, Q6K])
def test_dequantize_row_bit_exact(gpu, oracle_mod, qtype):
    P, O = gpu, oracle_mod
    rng = np.random.default_rng(qtype)
    for n in (256, 2048, 5632):
        for scale_exp in ((-14, -6), (2, 10)):
            rows = S.random_weights(rng, qtype, n, 3, scale_exp)
            dr = P.DeviceBuffer.from_numpy(rows)
            out = P.DeviceBuffer(4 * n)
            for r in range(3):
                rb = rows.shape[1]
                P.check(P.lib.plh_dequantize_row(qtype, dr.ptr + r * rb, out.ptr, n),
                        "plh_dequantize_row")
                want = O.dequantize(rows[r], n, 1, qtype)[0]
                got = out.download(np.float32, (n,))
                assert np.array_equal(bits(got), bits(want)), (qtype, n, r)


def test_dequantize_row_rejects(gpu):
    P = gpu
    b = P.DeviceBuffer(4096)
    assert P.lib.plh_dequantize_row(Q4K, b.ptr, b.ptr, 100) == -1      # not whole blocks
    assert P.lib.plh_dequantize_row(11, b.ptr, b.ptr, 256) == -1       # Q3_K: no kernel


@pytest.mark.parametrize("qtype,n,d", [(Q4K, 2048, 2048), (Q6K, 5632, 2048), (Q8, 2048, 256)])
def test_gemv_epilogues(gpu, oracle_mod, qtype, n, d):
    with gemv_order(gpu, "exact"):
        _gemv_epilogues_exact(gpu, oracle_mod, qtype, n, d)


@pytest.mark.parametrize("qtype,n,d", [(Q4K, 2048, 2048), (Q6K, 5632, 2048), (Q8, 2048, 256)])
def test_gemv_epilogues_fast_order(gpu, oracle_mod, qtype, n, d):
    """The fast order with each prologue / epilogue: within 128 fp32 ulps of
    sum |w xn| (both orders meet 64 of the float64 product; the rmsnorm's
    squares are summed as a tree) plus the epilogue's own rounding."""
    from test_gpu_gemv import decode64
    P, O = gpu, oracle_mod
    rng = np.random.default_rng(n + d + 1)
    W = S.random_weights(rng, qtype, n, d, S.unit_scale_exp(qtype, n))
    W64 = np.abs(decode64(qtype, W, n, d))
    x = rng.standard_normal(n).astype(np.float32)
    bias = rng.standard_normal(d).astype(np.float32)
    resid = rng.standard_normal(d).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, n).astype(np.float32)
    G = P.QMatrix(qtype, n, d, W)
    dx, db, dr, dnw = (P.DeviceBuffer.from_numpy(a) for a in (x, bias, resid, nw))
    out = P.DeviceBuffer(4 * d)
    vp = C.c_void_p
    eps32 = np.finfo(np.float32).eps
    for norm in (False, True):
        xn = O.rmsnorm(x, nw, 1e-5) if norm else x
        mag = W64 @ np.abs(xn.astype(np.float64))
        want = O.matmul(W, xn, n, d, qtype)
        for b, r in ((None, None), (db, None), (db, dr)):
            P.check(P.lib.plh_gemv_ex(qtype, n, d, vp(G.ptr), vp(dx.ptr), vp(out.ptr),
                                      vp(dnw.ptr) if norm else None, C.c_float(1e-5),
                                      vp(b.ptr) if b is not None else None, 0, None,
                                      vp(r.ptr) if r is not None else None), "plh_gemv_ex")
            got = out.download(np.float32, (d,)).astype(np.float64)
            ref = want.astype(np.float64)
            if b is not None:
                ref = ref + bias
            if r is not None:
                ref = ref + resid
            tol = 128 * eps32 * mag + 4 * eps32 * np.abs(ref) + 1e-30
            assert np.all(np.abs(got - ref) <= tol), (norm, b is None, r is None,
                                                      float(np.max(np.abs(got - ref) / tol)))


def _gemv_epilogues_exact(gpu, oracle_mod, qtype, n, d):
    P, O = gpu, oracle_mod
    rng = np.random.default_rng(n + d)
    W = S.random_weights(rng, qtype, n, d, S.unit_scale_exp(qtype, n))
    x = rng.standard_normal(n).astype(np.float32)
    bias = rng.standard_normal(d).astype(np.float32)
    resid = rng.standard_normal(d).astype(np.float32)
    gate = (rng.standard_normal(d) * 4).astype(np.float32)
    dot = O.matmul(W, x, n, d, qtype)
    G = P.QMatrix(qtype, n, d, W)
    dx = P.DeviceBuffer.from_numpy(x)
    db, dr = P.DeviceBuffer.from_numpy(bias), P.DeviceBuffer.from_numpy(resid)
    out = P.DeviceBuffer(4 * d)
    vp = C.c_void_p

    def run(b, bz, r, o, nw=None, eps=0.0):
        """plh_gemv_ex into buffer o; returns o's contents."""
        P.check(P.lib.plh_gemv_ex(qtype, n, d, vp(G.ptr), vp(dx.ptr), vp(o.ptr),
                                  nw and vp(nw.ptr), C.c_float(eps), b and vp(b.ptr), bz, None,
                                  r and vp(r.ptr)), "plh_gemv_ex")
        return o.download(np.float32, (d,))

    assert np.array_equal(bits(run(None, 0, None, out)), bits(dot))
    assert np.array_equal(bits(run(db, 0, None, out)), bits(dot + bias))
    assert np.array_equal(bits(run(None, 1, None, out)), bits(dot + np.float32(0.0)))
    # x = x + (dot + bias), in place on the residual
    assert np.array_equal(bits(run(db, 0, dr, dr)), bits(resid + (dot + bias)))
    # the rmsnorm prologue: W @ rmsnorm(x, w), bit-exact, with a bias
    nw = rng.uniform(0.5, 1.5, n).astype(np.float32)
    dnw = P.DeviceBuffer.from_numpy(nw)
    for eps in (1e-5, 1e-6):
        xn = O.rmsnorm(x, nw, eps)
        want = O.matmul(W, xn, n, d, qtype) + bias
        assert np.array_equal(bits(run(db, 0, None, out, dnw, eps)), bits(want)), eps
    # hb = silu(hb) * dot, in place on the gate: within the expf difference
    dg2 = P.DeviceBuffer.from_numpy(gate)
    P.check(P.lib.plh_gemv_ex(qtype, n, d, vp(G.ptr), vp(dx.ptr), vp(dg2.ptr), None,
                              C.c_float(0.0), None, 0, vp(dg2.ptr), None), "plh_gemv_ex")
    got = dg2.download(np.float32, (d,))
    silu = np.array([O.lib().orc_silu(float(v)) for v in gate], np.float32)
    want = silu * dot
    tol = 4 * np.spacing(np.abs(want)) + 1e-37
    assert np.all(np.abs(got - want) <= tol), np.max(np.abs(got - want) / tol)
    with pytest.raises(P.PicolmHipError):
        P.check(P.lib.plh_gemv_ex(qtype, n, d, vp(G.ptr), vp(dx.ptr), vp(out.ptr), None,
                                  C.c_float(0.0), vp(db.ptr), 1, None, None), "plh_gemv_ex")


LLAMA = dict(n_layers=3, n_embd=512, n_ffn=1024, n_heads=8, n_kv_heads=2, head_dim=64,
             vocab_size=1000, max_seq_len=256, rope_type=0, rope_base=1e4, eps=1e-5,
             types=dict(embd=Q4K, output=Q6K, q=Q4K, k=Q8, v=Q6K, o=Q4K, gate=Q4K, up=Q8,
                        down=Q6K))
QWEN = dict(n_layers=2, n_embd=512, n_ffn=768, n_heads=4, n_kv_heads=2, head_dim=128,
            vocab_size=700, max_seq_len=128, rope_type=1, rope_base=1e6, eps=1e-6,
            types=dict(embd=Q8, output=Q8, q=Q8, k=Q4K, v=Q6K, o=Q8, gate=Q6K, up=Q4K,
                       down=Q4K), biases=True, qk_norm=True)
# head dims without a tuned attention kernel (attn_generic.hip)
HD96 = dict(LLAMA, n_layers=2, n_embd=768, head_dim=96)
HD80_QKN = dict(QWEN, n_embd=1280, n_heads=16, n_kv_heads=4, head_dim=80)
MODELS = [LLAMA, QWEN, HD96, HD80_QKN]
MODEL_IDS = ["llama", "qwen", "llama_hd96", "qwen_hd80"]


def normwise(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.parametrize("order", ["exact", "fast"])
@pytest.mark.parametrize("cfg", MODELS, ids=MODEL_IDS)
def test_forward_matches_oracle(gpu, oracle_mod, cfg, order):
    with gemv_order(gpu, order):
        _forward_matches_oracle(gpu, oracle_mod, cfg, order == "exact")


def _forward_matches_oracle(gpu, oracle_mod, cfg, exact):
    P, O = gpu, oracle_mod
    h = S.SynthModel(**cfg, seed=11)
    dm = P.DeviceModel(h)
    orc = O.OracleForward(h)
    rng = np.random.default_rng(12)
    kv_layer = h.max_seq_len * h.kv_dim
    tol = FWD_TOL if exact else FWD_TOL_FAST
    worst = 0.0
    try:
        for pos in list(range(6)) + [40, 41]:
            tok = int(rng.integers(0, h.vocab_size))
            print(f"[case] forward {h.n_layers}x{h.n_embd} hd {h.head_dim} pos {pos} tok {tok}",
                  flush=True)
            dm.forward(tok, pos)
            P.synchronize()
            lg, x = dm.fetch_logits(), dm.fetch_x()
            lo, xo = orc.forward(tok, pos, n_threads=8)
            e = max(normwise(lg, lo), normwise(x, xo))
            worst = max(worst, e)
            assert e <= tol, (pos, e)
            top = np.argsort(lo)[-2:]
            if lo[top[1]] - lo[top[0]] > 4 * tol * np.max(np.abs(lo)):
                assert int(np.argmax(lg)) == int(top[1]), pos
            kc, vc = dm.fetch_cache()
            # layer 0's rows involve no transcendental: bit-exact in the exact
            # GEMV order (the fast order checks them with the later layers)
            first = kv_layer if exact else 0
            if exact:
                assert np.array_equal(kc[:kv_layer], orc.kc[:kv_layer]), pos
                assert np.array_equal(vc[:kv_layer], orc.vc[:kv_layer]), pos
            # later layers: inputs equal up to a normwise ~1e-6, so a value
            # may round to the neighbouring fp16 step, plus that input error
            for dev_bits, orc_bits in ((kc, orc.kc), (vc, orc.vc)):
                a = O.f16_to_f32(dev_bits[first:])
                b = O.f16_to_f32(orc_bits[first:])
                step = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16))
                kv_tol = KV_TOL if exact else KV_TOL_FAST
                bound = step.astype(np.float32) + kv_tol * np.max(np.abs(b))
                assert np.all(np.abs(a - b) <= bound), (pos, np.max(np.abs(a - b) / bound))
            # positions 6..39 are skipped: copy the oracle's rows over so both
            # caches agree (the reference's kvcache_load does the same)
            if pos == 5:
                dm.load_cache(orc.kc, orc.vc)
        print(f"forward {cfg['n_layers']} layers: worst normwise error {worst:.2e}")
    finally:
        dm.free()


@pytest.mark.parametrize("cfg", MODELS, ids=MODEL_IDS)
def test_prefill_matches_oracle(gpu, oracle_mod, cfg):
    """model_forward_prefill: chunks of a prompt over a cached prefix, then a
    decode step; logits of each chunk's last token, layer-0 KV rows exact."""
    P, O = gpu, oracle_mod
    h = S.SynthModel(**cfg, seed=21)
    dm = P.DeviceModel(h)
    orc = O.OracleForward(h)
    rng = np.random.default_rng(22)
    kv_layer = h.max_seq_len * h.kv_dim
    try:
        start = 0
        for n in (7, 1, 12):
            toks = rng.integers(0, h.vocab_size, n).astype(np.int32)
            print(f"[case] prefill {h.n_layers}x{h.n_embd} start {start} n {n}", flush=True)
            dm.prefill(toks, start)
            P.synchronize()
            lo, xo = orc.prefill(toks, start, n_threads=8)
            # the last token's rmsnorm and logits run in the default (fast) order
            assert max(normwise(dm.fetch_logits(), lo), normwise(dm.fetch_x(), xo)) <= FWD_TOL_FAST
            kc, vc = dm.fetch_cache()
            assert np.array_equal(kc[:kv_layer], orc.kc[:kv_layer]), start
            assert np.array_equal(vc[:kv_layer], orc.vc[:kv_layer]), start
            start += n
        dm.forward(5, start)
        P.synchronize()
        lo, xo = orc.forward(5, start, n_threads=8)
        assert normwise(dm.fetch_logits(), lo) <= FWD_TOL_FAST
        with pytest.raises(P.PicolmHipError):
            dm.prefill([1, 2], h.max_seq_len - 1)
        with pytest.raises(P.PicolmHipError):
            dm.prefill([h.vocab_size], 0)
    finally:
        dm.free()


def test_prefill_long_prompt_chunks(gpu, oracle_mod):
    """A 200-token prompt after a 5-token prefix: two 128-token chunks (the
    second ragged), embedding launches of 64 tokens, then a decode step."""
    P, O = gpu, oracle_mod
    h = S.SynthModel(**dict(LLAMA, n_layers=2, max_seq_len=256), seed=43)
    dm = P.DeviceModel(h)
    orc = O.OracleForward(h)
    rng = np.random.default_rng(44)
    kv_layer = h.max_seq_len * h.kv_dim
    try:
        start = 0
        for n in (5, 200):
            toks = rng.integers(0, h.vocab_size, n).astype(np.int32)
            print(f"[case] long prefill start {start} n {n}", flush=True)
            dm.prefill(toks, start)
            P.synchronize()
            lo, xo = orc.prefill(toks, start, n_threads=8)
            assert max(normwise(dm.fetch_logits(), lo), normwise(dm.fetch_x(), xo)) <= FWD_TOL_FAST
            start += n
        kc, vc = dm.fetch_cache()
        assert np.array_equal(kc[:kv_layer], orc.kc[:kv_layer])
        assert np.array_equal(vc[:kv_layer], orc.vc[:kv_layer])
        dm.forward(9, start)
        P.synchronize()
        lo, _ = orc.forward(9, start, n_threads=8)
        assert normwise(dm.fetch_logits(), lo) <= FWD_TOL_FAST
    finally:
        dm.free()


def test_forward_separate_norm_launches(gpu, oracle_mod):
    """Tuning key 4 forms each rmsnorm in a launch of its own (the path of
    n_embd > 7680): same logits and state.x as the fused prologue (in the
    exact GEMV order, whose fused rmsnorm is the reference's)."""
    P, O = gpu, oracle_mod
    h = S.SynthModel(**dict(LLAMA, n_layers=2), seed=41)
    dm = P.DeviceModel(h)
    P.check(P.lib.plh_set_tuning(10, 1), "plh_set_tuning")
    try:
        got = {}
        for mode in (0, 1):
            P.check(P.lib.plh_set_tuning(4, mode), "plh_set_tuning")
            dm.load_cache(np.zeros(h.cache_elems(), np.uint16), np.zeros(h.cache_elems(), np.uint16))
            for pos, tok in enumerate((5, 6, 7)):
                dm.forward(tok, pos)
            P.synchronize()
            got[mode] = (dm.fetch_logits(), dm.fetch_x())
        assert np.array_equal(got[0][0].view(np.uint32), got[1][0].view(np.uint32))
        assert np.array_equal(got[0][1].view(np.uint32), got[1][1].view(np.uint32))
    finally:
        P.check(P.lib.plh_set_tuning(4, 0), "plh_set_tuning")
        P.check(P.lib.plh_set_tuning(10, 0), "plh_set_tuning")
        dm.free()


def test_forward_rejects_bad_calls(gpu):
    P = gpu
    h = S.SynthModel(**dict(LLAMA, n_layers=1), seed=13)
    dm = P.DeviceModel(h)
    try:
        for tok, pos in ((-1, 0), (h.vocab_size, 0), (0, -1), (0, h.max_seq_len)):
            with pytest.raises(P.PicolmHipError):
                dm.forward(tok, pos)
        # a matrix type the GEMV has no kernel for: nothing is queued
        saved = dm.layers[0].up.qtype
        dm.layers[0].up.qtype = F32
        with pytest.raises(P.PicolmHipError, match="GEMV-capable"):
            dm.forward(0, 0)
        dm.layers[0].up.qtype = saved
        dm.layers[0].k_norm = dm.layers[0].attn_norm   # only one of the QK-norm pair
        with pytest.raises(P.PicolmHipError, match="q_norm"):
            dm.forward(0, 0)
    finally:
        dm.free()


# gate and up of one type, so that they run (and are prefetched) as a pair
PF_LLAMA = dict(LLAMA, n_layers=2, max_seq_len=2048, types=dict(LLAMA["types"], up=Q4K))
PF_QWEN = dict(QWEN, max_seq_len=2048, types=dict(QWEN["types"], up=Q6K))


@pytest.mark.parametrize("cfg", [PF_LLAMA, PF_QWEN], ids=["llama", "qwen"])
def test_forward_weight_prefetch_changes_nothing(gpu, cfg):
    """Tuning key 15: the attention launch's spare workgroups that load the
    next GEMVs' weights into the L2 (every setting) leave every result
    bit-identical to no prefetch: logits, residual and both caches, at a
    short position (unsplit attention launch) and past 512 positions (split
    or stream-K launch)."""
    P = gpu
    h = S.SynthModel(**cfg, seed=71)
    dm = P.DeviceModel(h)
    rng = np.random.default_rng(72)
    fill = rng.standard_normal((2, h.cache_elems()), dtype=np.float32).astype(np.float16)
    kc, vc = fill[0].view(np.uint16), fill[1].view(np.uint16)
    try:
        for pos in (100, 1500, 2047):
            ref = None
            for key in (-1, 0, 1):
                P.check(P.lib.plh_set_tuning(15, key), "plh_set_tuning")
                dm.load_cache(kc, vc)
                print(f"[case] forward prefetch setting {key} pos {pos}", flush=True)
                dm.forward(7, pos)
                P.synchronize()
                got = (bits(dm.fetch_logits()), bits(dm.fetch_x())) + tuple(dm.fetch_cache())
                if ref is None:
                    ref = got
                    continue
                for a, b in zip(ref, got):
                    assert np.array_equal(a, b), (pos, key)
    finally:
        P.check(P.lib.plh_set_tuning(15, 0), "plh_set_tuning")
        dm.free()


# head_dim 128 without QK-norm: the fused q/k/v + attention launch's other shape
PF_LLAMA128 = dict(PF_LLAMA, n_heads=4, n_kv_heads=2, head_dim=128)
# Qwen's rope pairing and q/k/v biases without QK-norm; one q head per kv head;
# 16 q heads per kv head (the most one head block takes)
PF_QWENROPE = dict(PF_LLAMA, rope_type=1, rope_base=1e6, biases=True)
PF_G1 = dict(PF_LLAMA, n_heads=4, n_kv_heads=4, head_dim=64, n_embd=256)
PF_G16 = dict(PF_LLAMA, n_heads=16, n_kv_heads=1, head_dim=64, n_embd=1024)


@pytest.mark.parametrize("cfg", [PF_LLAMA, PF_LLAMA128, PF_QWENROPE, PF_G1, PF_G16],
                         ids=["hd64", "hd128", "qwen_rope_bias", "g1", "g16"])
def test_forward_fused_qkv_attention_changes_nothing(gpu, cfg):
    """Tuning key 17: q, k, v and the attention in one launch (the attention
    workgroups wait on per-group counts of the GEMV workgroups that stored
    their rows) give the bits of the two launches -- logits, residual and
    both caches -- with every prefetch count, at a short position (fused)
    and past 512 positions (not fused), several tokens in a row."""
    P = gpu
    h = S.SynthModel(**cfg, seed=73)
    dm = P.DeviceModel(h)
    rng = np.random.default_rng(74)
    fill = rng.standard_normal((2, h.cache_elems()), dtype=np.float32).astype(np.float16)
    kc, vc = fill[0].view(np.uint16), fill[1].view(np.uint16)
    try:
        for pos in (100, 511, 1500):
            ref = None
            for key in (-1, 0, 8, 31):
                P.check(P.lib.plh_set_tuning(17, key), "plh_set_tuning")
                dm.load_cache(kc, vc)
                print(f"[case] forward fusion setting {key} pos {pos}", flush=True)
                for i in range(3):
                    dm.forward(7 + i, pos + i if pos + i < h.max_seq_len else pos)
                P.synchronize()
                got = (bits(dm.fetch_logits()), bits(dm.fetch_x())) + tuple(dm.fetch_cache())
                if ref is None:
                    ref = got
                    continue
                for a, b in zip(ref, got):
                    assert np.array_equal(a, b), (pos, key)
    finally:
        P.check(P.lib.plh_set_tuning(17, 0), "plh_set_tuning")
        dm.free()


@pytest.mark.parametrize("cfg", [dict(LLAMA, n_layers=2, max_seq_len=2048),
                                 dict(QWEN, max_seq_len=2048)], ids=["llama", "qwen"])
def test_forward_long_context_split_decode(gpu, oracle_mod, cfg):
    """Decode steps past 512 cached positions, where the attention launch is
    split across workgroups and merged, and the workspace grows: caches
    pre-filled with N(0,1) rows rounded to fp16 (what kvcache_load would
    bring in), then model_forward at 600, 601 and 2047 (the last cache row),
    logits, residual and appended rows against the oracle."""
    P, O = gpu, oracle_mod
    h = S.SynthModel(**cfg, seed=61)
    dm = P.DeviceModel(h)
    orc = O.OracleForward(h)
    rng = np.random.default_rng(62)
    kv_layer = h.max_seq_len * h.kv_dim
    try:
        for fill, steps in ((600, (600, 601)), (2047, (2047,))):
            kc = np.zeros(h.cache_elems(), np.uint16)
            vc = np.zeros(h.cache_elems(), np.uint16)
            for l in range(h.n_layers):
                rows = slice(l * kv_layer, l * kv_layer + fill * h.kv_dim)
                kc[rows] = O.f32_to_f16(rng.standard_normal(fill * h.kv_dim).astype(np.float32))
                vc[rows] = O.f32_to_f16(rng.standard_normal(fill * h.kv_dim).astype(np.float32))
            orc.kc[:] = kc      # the oracle model holds these arrays' addresses
            orc.vc[:] = vc
            dm.load_cache(kc, vc)
            for pos in steps:
                tok = int(rng.integers(0, h.vocab_size))
                print(f"[case] long-context forward {h.n_layers}x{h.n_embd} pos {pos} tok {tok}",
                      flush=True)
                dm.forward(tok, pos)
                P.synchronize()
                lo, xo = orc.forward(tok, pos, n_threads=8)
                e = max(normwise(dm.fetch_logits(), lo), normwise(dm.fetch_x(), xo))
                assert e <= FWD_TOL_FAST, (pos, e)
                gk, gv = dm.fetch_cache()
                # the default fast GEMV order: every layer's rows within one
                # fp16 step plus the input error
                for dev_bits, orc_bits in ((gk, orc.kc), (gv, orc.vc)):
                    a = O.f16_to_f32(dev_bits)
                    b = O.f16_to_f32(orc_bits)
                    step = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16))
                    bound = step.astype(np.float32) + KV_TOL_FAST * np.max(np.abs(b))
                    assert np.all(np.abs(a - b) <= bound), pos
                # keep both caches identical for the next step
                dm.load_cache(orc.kc, orc.vc)
    finally:
        dm.free()
