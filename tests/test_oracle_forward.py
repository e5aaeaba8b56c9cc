"""Pins the oracle's whole forward pass (forward_oracle.c) -- what the device
forward is checked against -- against the reference's own model_forward and
model_forward_prefill (model.c:742-925, 939-1144, compiled into oracle/_ref
and driven by ref_harness.c on the same host buffers).

Checks: logits, the final normalised residual and both KV caches bit-exact
after every decode step and every prefill chunk, for a LLaMA-shaped model
with mixed Q4_K / Q6_K / Q8_0 matrices and a Qwen-shaped one (half-split
RoPE, q/k/v/o biases, QK-norm, F32 matrices); every embedding type; silu
against float64; and, without the reference, a model whose layers add
exact zeros reducing to rmsnorm(embedding row) @ output.
"""
import numpy as np
import pytest

from conftest import needs_ref
from picolm_amd import synth as S

Q4K, Q6K, Q8, F32, F16 = S.TYPE_Q4_K, S.TYPE_Q6_K, S.TYPE_Q8_0, S.TYPE_F32, S.TYPE_F16

LLAMA = dict(n_layers=2, n_embd=256, n_ffn=512, n_heads=4, n_kv_heads=2, head_dim=64,
             vocab_size=300, max_seq_len=64, rope_type=0, rope_base=1e4, eps=1e-5,
             types=dict(embd=Q4K, output=Q6K, q=Q4K, k=Q8, v=Q6K, o=Q4K, gate=Q4K, up=Q8,
                        down=Q6K))
QWEN = dict(n_layers=2, n_embd=256, n_ffn=256, n_heads=2, n_kv_heads=1, head_dim=128,
            vocab_size=200, max_seq_len=32, rope_type=1, rope_base=1e6, eps=1e-6,
            types=dict(embd=Q8, output=Q8, q=F32, k=Q8, v=Q4K, o=Q8, gate=F32, up=Q6K,
                       down=Q4K), biases=True, qk_norm=True)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_same(O_pair, R_pair, what):
    (lo, xo), (lr, xr) = O_pair, R_pair
    assert np.array_equal(bits(lo), bits(lr)), f"{what}: logits differ"
    assert np.array_equal(bits(xo), bits(xr)), f"{what}: final residual differs"


@needs_ref
@pytest.mark.parametrize("cfg", [LLAMA, QWEN], ids=["llama", "qwen"])
def test_decode_matches_reference_bits(oracle_mod, cfg):
    O = oracle_mod
    h = S.SynthModel(**cfg, seed=3)
    orc, ref = O.OracleForward(h), O.RefForward(h)
    rng = np.random.default_rng(5)
    try:
        for pos in range(10):
            tok = int(rng.integers(0, h.vocab_size))
            assert_same(orc.forward(tok, pos, n_threads=1 + pos % 3), ref.forward(tok, pos),
                        f"pos {pos}")
            assert np.array_equal(orc.kc, ref.kc) and np.array_equal(orc.vc, ref.vc), pos
    finally:
        ref.close()


@needs_ref
@pytest.mark.parametrize("cfg", [LLAMA, QWEN], ids=["llama", "qwen"])
def test_prefill_matches_reference_bits(oracle_mod, cfg):
    O = oracle_mod
    h = S.SynthModel(**cfg, seed=4)
    orc, ref = O.OracleForward(h), O.RefForward(h)
    rng = np.random.default_rng(6)
    try:
        start = 0
        for n in (5, 1, 7):   # chunks, the later ones over a cached prefix
            toks = rng.integers(0, h.vocab_size, n).astype(np.int32)
            assert_same(orc.prefill(toks, start, n_threads=2), ref.prefill(toks, start),
                        f"chunk at {start}")
            assert np.array_equal(orc.kc, ref.kc) and np.array_equal(orc.vc, ref.vc), start
            start += n
        # a decode step after the prompt continues from the same caches
        assert_same(orc.forward(7, start), ref.forward(7, start), "decode after prefill")
    finally:
        ref.close()


@needs_ref
@pytest.mark.parametrize("embd", [F32, F16, Q8, Q4K, Q6K])
def test_embedding_types_match_reference(oracle_mod, embd):
    O = oracle_mod
    cfg = dict(LLAMA, types=dict(LLAMA["types"], embd=embd), n_layers=1)
    h = S.SynthModel(**cfg, seed=7)
    orc, ref = O.OracleForward(h), O.RefForward(h)
    try:
        for pos, tok in enumerate((0, h.vocab_size - 1, 17)):
            assert_same(orc.forward(tok, pos), ref.forward(tok, pos), f"embd {embd} pos {pos}")
    finally:
        ref.close()


def test_silu_against_float64(oracle_mod):
    O = oracle_mod
    # where expf(-x) is finite in fp32: within 3 ulps of float64
    x = np.concatenate([np.linspace(-88, 90, 4001), [-1e-30, 0.0, 1e-30, 88.7]])
    x = x.astype(np.float32)
    got = np.array([O.lib().orc_silu(float(v)) for v in x], np.float32)
    x64 = x.astype(np.float64)
    want = x64 / (1.0 + np.exp(-x64))
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 3 * ulp)
    # below about -88.7 expf(-x) overflows to inf and x / inf is -0
    for v in (-89.0, -103.0, -1e4):
        r = np.float32(O.lib().orc_silu(v))
        assert r == 0.0 and np.signbit(r)


@needs_ref
def test_silu_matches_reference_bits(oracle_mod):
    O = oracle_mod
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(20000) * 6).astype(np.float32)
    want = x.copy()
    O.ref().ref_silu(want, len(want))
    got = np.array([O.lib().orc_silu(float(v)) for v in x], np.float32)
    assert np.array_equal(bits(got), bits(want))


def test_zero_layers_reduce_to_norm_and_output(oracle_mod):
    """With every o and down scale zero the layers add exact zeros to the
    residual, so the logits are output @ rmsnorm(embedding row)."""
    O = oracle_mod
    h = S.SynthModel(**dict(LLAMA, types=dict(LLAMA["types"], o=Q8, down=Q8)), seed=9)
    for L in h.layers:
        for name in ("o", "down"):
            qt, rows = L[name]
            rows = rows.copy()
            rows.reshape(rows.shape[0], -1, 34)[:, :, 0:2] = 0   # every block scale = 0
            L[name] = (qt, rows)
    orc = O.OracleForward(h)
    for pos, tok in enumerate((3, 250)):
        logits, x = orc.forward(tok, pos)
        e = O.dequantize(h.token_embd[tok], h.n_embd, 1, h.embd_type)[0]
        xn = O.rmsnorm(e, h.output_norm, h.eps)
        assert np.array_equal(bits(x), bits(xn))
        want = O.matmul(h.output, xn, h.n_embd, h.vocab_size, h.output_type)
        assert np.array_equal(bits(logits), bits(want))


def test_bad_arguments_rejected(oracle_mod):
    O = oracle_mod
    h = S.SynthModel(**LLAMA, seed=10)
    orc = O.OracleForward(h)
    for tok, pos in ((-1, 0), (h.vocab_size, 0), (0, -1), (0, h.max_seq_len)):
        with pytest.raises(ValueError):
            orc.forward(tok, pos)
    with pytest.raises(ValueError):
        orc.prefill([1, 2, 3], h.max_seq_len - 2)


@needs_ref
def test_tinyllama_shape_matches_reference_bits(oracle_mod):
    """The full TinyLlama-1.1B Q4_K_M shape (22 layers, n_embd 2048, n_ffn
    5632, GQA 32/4, vocab 32000; layer bytes shared): two decode steps."""
    O = oracle_mod
    h = S.SynthModel(22, 2048, 5632, 32, 4, 64, 32000, 2048, seed=7, share_layers=True)
    orc, ref = O.OracleForward(h), O.RefForward(h)
    O.ref().ref_set_threads(4)
    try:
        for pos, tok in enumerate((1, 31999)):
            assert_same(orc.forward(tok, pos, n_threads=8), ref.forward(tok, pos), f"pos {pos}")
        assert np.array_equal(orc.kc, ref.kc) and np.array_equal(orc.vc, ref.vc)
    finally:
        O.ref().ref_set_threads(1)
        ref.close()
