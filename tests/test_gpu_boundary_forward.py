"""gpu_try_forward / gpu_try_forward_prefill (gpu_hip.c) on the GPU, driven
from C by tests/c/test_gpu_forward the way picolm's model_forward and
model_forward_prefill would call them, against the oracle's forward pass.

Checks: a prompt in two prefill chunks then decode steps returns 0 each
time; logits and state.x match the oracle's within the forward tolerance;
the host caches hold the appended rows (layer 0 bit-exact, later layers to
one fp16 step); PICOLM_HIP_FORWARD=0, a model with an F32 projection, models
whose q_dim is not n_embd and PICOLM_GPU_LAYERS below the layer count fall
back (-1, nothing written)."""
import os
import subprocess

import numpy as np
import pytest

from attn_check import FWD_TOL, FWD_TOL_FAST, KV_TOL, KV_TOL_FAST
from conftest import ROOT
from picolm_amd import synth as S

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "c", "test_gpu_forward")
Q4K, Q6K, Q8, F32 = S.TYPE_Q4_K, S.TYPE_Q6_K, S.TYPE_Q8_0, S.TYPE_F32
LAYER = ("q", "k", "v", "o", "gate", "up", "down")


def write_model(f, h):
    has_bias = h.layers[0]["q_bias"] is not None
    has_qkn = h.layers[0]["q_norm"] is not None
    np.array([h.n_layers, h.n_embd, h.n_ffn, h.n_heads, h.n_kv_heads, h.head_dim, h.vocab_size,
              h.max_seq_len, h.rope_type], np.int32).tofile(f)
    np.array([h.eps, h.rope_base], np.float32).tofile(f)
    types = [h.embd_type, h.output_type]
    for L in h.layers:
        types += [L[name][0] for name in LAYER]
    np.array(types, np.int32).tofile(f)
    np.array([has_bias, has_qkn], np.int32).tofile(f)
    h.token_embd.tofile(f)
    h.output_norm.tofile(f)
    h.output.tofile(f)
    for L in h.layers:
        L["attn_norm"].tofile(f)
        L["ffn_norm"].tofile(f)
        for name in LAYER:
            L[name][1].tofile(f)
        if has_bias:
            for name in ("q_bias", "k_bias", "v_bias", "o_bias"):
                L[name].tofile(f)
        if has_qkn:
            L["q_norm"].tofile(f)
            L["k_norm"].tofile(f)


def run(tmp_path, h, steps, env_extra=None):
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        write_model(f, h)
        np.array([len(steps)], np.int32).tofile(f)
        for kind, start, toks in steps:
            np.array([kind, start, len(toks)] + list(toks), np.int32).tofile(f)
    env = dict(os.environ)
    env["PICOLM_HIP_GEMV_EXACT"] = "1"   # the exact GEMV order unless a test asks otherwise
    env.update(env_extra or {})
    print(f"[case] boundary forward {h.n_layers}x{h.n_embd} steps {len(steps)} env {env_extra}",
          flush=True)
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
    rcs = tuple(int(v) for v in take(np.int32, 2))
    res = []
    for _ in steps:
        rc = int(take(np.int32, 1)[0])
        res.append((rc, take(np.float32, h.vocab_size), take(np.float32, h.n_embd)))
    n = h.cache_elems()
    return rcs, res, take(np.uint16, n), take(np.uint16, n)


def normwise(a, b):
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


CFG = dict(n_layers=2, n_embd=512, n_ffn=1024, n_heads=8, n_kv_heads=2, head_dim=64,
           vocab_size=600, max_seq_len=64, rope_type=0, rope_base=1e4, eps=1e-5,
           types=dict(embd=Q6K, output=Q8, q=Q4K, k=Q4K, v=Q6K, o=Q8, gate=Q4K, up=Q4K,
                      down=Q6K))
QWEN = dict(CFG, rope_type=1, rope_base=1e6, eps=1e-6, head_dim=128, n_heads=4,
            biases=True, qk_norm=True, types=dict(CFG["types"], embd=Q8, gate=Q6K, up=Q4K))


@pytest.mark.parametrize("order", ["exact", "fast"])
@pytest.mark.parametrize("cfg", [CFG, QWEN], ids=["llama", "qwen"])
def test_forward_through_boundary(tmp_path, oracle_mod, cfg, order):
    """In the exact GEMV order (PICOLM_HIP_GEMV_EXACT=1) layer 0's rows are
    bit-exact; in the default fast order every layer's rows are within one
    fp16 step plus the input error."""
    O = oracle_mod
    h = S.SynthModel(**cfg, seed=31)
    rng = np.random.default_rng(32)
    p1 = rng.integers(0, h.vocab_size, 6).tolist()
    p2 = rng.integers(0, h.vocab_size, 3).tolist()
    steps = [(1, 0, p1), (1, 6, p2), (0, 9, [17]), (0, 10, [h.vocab_size - 1])]
    exact = order == "exact"
    rcs, res, kc, vc = run(tmp_path, h, steps, {"PICOLM_HIP_GEMV_EXACT": "1" if exact else "0"})
    assert rcs == (0, 0)
    orc = O.OracleForward(h)
    tol = FWD_TOL if exact else FWD_TOL_FAST
    for (kind, start, toks), (rc, lg, x) in zip(steps, res):
        assert rc == 0, (kind, start)
        lo, xo = orc.prefill(toks, start, 8) if kind else orc.forward(toks[0], start, 8)
        assert max(normwise(lg, lo), normwise(x, xo)) <= tol, (kind, start)
    kv_layer = h.max_seq_len * h.kv_dim
    first = kv_layer if exact else 0
    if exact:
        assert np.array_equal(kc[:kv_layer], orc.kc[:kv_layer])
        assert np.array_equal(vc[:kv_layer], orc.vc[:kv_layer])
    kv_tol = KV_TOL if exact else KV_TOL_FAST
    for dev_bits, orc_bits in ((kc, orc.kc), (vc, orc.vc)):
        a, b = O.f16_to_f32(dev_bits[first:]), O.f16_to_f32(orc_bits[first:])
        step = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16)).astype(np.float32)
        assert np.all(np.abs(a - b) <= step + kv_tol * np.max(np.abs(b)))


def test_forward_fallbacks(tmp_path):
    steps = [(0, 0, [3]), (1, 1, [4, 5])]
    h = S.SynthModel(**CFG, seed=33)
    for env in ({"PICOLM_HIP_FORWARD": "0"}, {"PICOLM_GPU_LAYERS": "1"}):
        rcs, res, kc, vc = run(tmp_path, h, steps, env)
        assert rcs == (0, 0)
        for rc, lg, x in res:
            assert rc == -1 and not lg.any() and not x.any()
        assert not kc.any() and not vc.any()
    h32 = S.SynthModel(**dict(CFG, types=dict(CFG["types"], down=F32)), seed=34)
    rcs, res, kc, vc = run(tmp_path, h32, steps)
    assert rcs == (0, 0)
    assert all(rc == -1 for rc, _, _ in res)
    # q_dim = n_heads * head_dim other than n_embd: the reference's loader
    # never builds one (head_dim = n_embd / n_heads, model.c:408), so the
    # whole-forward hooks decline and the CPU path runs
    for heads, seed in ((16, 35), (4, 36)):
        hq = S.SynthModel(**dict(CFG, n_heads=heads, n_kv_heads=2,
                                 types=dict(CFG["types"], o=Q8)), seed=seed)
        rcs, res, kc, vc = run(tmp_path, hq, steps)
        assert rcs == (0, 0)
        assert all(rc == -1 and not lg.any() for rc, lg, _ in res)


@pytest.mark.parametrize("cfg", [CFG, QWEN], ids=["llama", "qwen"])
def test_forward_through_boundary_long_context(tmp_path, oracle_mod, cfg):
    """Decode past 512 cached positions through gpu_try_forward, where the
    attention launch is split and merged and the logits, state.x and rows
    come back through pinned staging: a 600-token prompt, decode at 600 and
    601, the prompt continued to position 2046, decode at 2047 (the last
    cache row)."""
    O = oracle_mod
    h = S.SynthModel(**dict(cfg, max_seq_len=2048), seed=37)
    rng = np.random.default_rng(38)
    toks = lambda n: rng.integers(0, h.vocab_size, n).tolist()
    steps = [(1, 0, toks(600)), (0, 600, toks(1)), (0, 601, toks(1)), (1, 602, toks(1445)),
             (0, 2047, toks(1))]
    rcs, res, kc, vc = run(tmp_path, h, steps, {"PICOLM_HIP_GEMV_EXACT": "0"})
    assert rcs == (0, 0)
    orc = O.OracleForward(h)
    for (kind, start, tk), (rc, lg, x) in zip(steps, res):
        assert rc == 0, (kind, start)
        lo, xo = orc.prefill(tk, start, 16) if kind else orc.forward(tk[0], start, 16)
        assert max(normwise(lg, lo), normwise(x, xo)) <= FWD_TOL_FAST, (kind, start)
    # the fast GEMV order: every layer's rows within one fp16 step plus the
    # input error (the prompt's rows come from the exact batched GEMVs)
    for dev_bits, orc_bits in ((kc, orc.kc), (vc, orc.vc)):
        a, b = O.f16_to_f32(dev_bits), O.f16_to_f32(orc_bits)
        step = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16)).astype(np.float32)
        assert np.all(np.abs(a - b) <= step + KV_TOL_FAST * np.max(np.abs(b)))
