"""Pins the oracle's weight GEMV (gpu_try_matmul's path: quant.c's fused
dequantize + dot products, tensor.c's matmul row loop).

Checks:
  * bit-exact against the reference's own vec_dot_q4_K/q6_K/q8_0/f32 and
    dequantize_row (quant.c compiled into oracle/_ref for x86-64 with AVX2,
    as the GPU host's native build), over random blocks of every field and
    the model's row lengths;
  * against float64 dequantize-then-dot within a bound of a few fp32 ulps
    of sum |w*x| (a dropped min term, a wrong nibble, a transposed scale or a
    skipped block fails it without the reference);
  * known answers from hand-built blocks (unit scales, constant quants).
"""
import numpy as np
import pytest

from conftest import needs_ref
from picolm_amd import synth as S

TYPES = {"q4_K": 12, "q6_K": 14, "q8_0": 8, "f32": 0}
ROW_LENS = {"q4_K": [256, 512, 2048, 5632], "q6_K": [256, 2048, 5632],
            "q8_0": [32, 96, 2048, 5632], "f32": [7, 16, 100, 2048]}


def _rows(O, rng, name, n, d, scale_exp=(-12, -4)):
    return S.random_weights(rng, TYPES[name], n, d, scale_exp)


@needs_ref
@pytest.mark.parametrize("name", list(TYPES))
def test_vec_dot_matches_reference_bits(oracle_mod, name):
    O = oracle_mod
    R = O.ref()
    ref_dot = getattr(R, f"vec_dot_{name}_f32")
    rng = np.random.default_rng(TYPES[name] + 1)
    for n in ROW_LENS[name]:
        for scale_exp in ((-14, -6), (-6, 2), (2, 10)):
            d = 24
            W = _rows(O, rng, name, n, d, scale_exp)
            x = (rng.standard_normal(n) * 10.0 ** rng.uniform(-2, 2)).astype(np.float32)
            got = O.matmul(W, x, n, d, TYPES[name])
            want = np.array([ref_dot(np.ascontiguousarray(W[i]), x, n) for i in range(d)],
                            np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n, scale_exp)
            # the reference's generic dispatch gives the same
            disp = np.array([R.vec_dot(np.ascontiguousarray(W[i]), x, n, TYPES[name])
                             for i in range(d)], np.float32)
            assert np.array_equal(disp.view(np.uint32), want.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("name", ["q4_K", "q6_K", "q8_0"])
def test_dequantize_matches_reference_bits(oracle_mod, name):
    O = oracle_mod
    R = O.ref()
    rng = np.random.default_rng(7)
    n, d = 512, 16
    W = _rows(O, rng, name, n, d)
    got = O.dequantize(W, n, d, TYPES[name])
    for i in range(d):
        want = np.empty(n, np.float32)
        R.dequantize_row(np.ascontiguousarray(W[i]), want, n, TYPES[name])
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), i


@pytest.mark.parametrize("name", list(TYPES))
def test_vec_dot_matches_float64(oracle_mod, name):
    """The fused dot equals dequantize-then-dot in float64 up to fp32 rounding
    of the partial sums; the dequantized weights are checked against an
    independent numpy decoding of the block fields."""
    O = oracle_mod
    rng = np.random.default_rng(11)
    n = 2048 if name != "f32" else 1000
    d = 32
    W = _rows(O, rng, name, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    got = O.matmul(W, x, n, d, TYPES[name]).astype(np.float64)
    w64 = _decode64(name, W, n, d)
    exact = w64 @ x.astype(np.float64)
    bound = 64 * np.finfo(np.float32).eps * (np.abs(w64) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound + 1e-30), np.max(np.abs(got - exact) / bound)
    # the oracle's dequantize agrees with the numpy decoding to fp32 rounding
    deq = O.dequantize(W, n, d, TYPES[name]).astype(np.float64)
    assert np.allclose(deq, w64, rtol=2 * np.finfo(np.float32).eps, atol=0)


def _decode64(name, W, n, d):
    """float64 weights from the block fields, written from the format
    description (quant.h:66-125) independently of the C code."""
    if name == "f32":
        return W.view(np.float32).reshape(d, n).astype(np.float64)
    if name == "q8_0":
        b = W.reshape(d, n // 32, 34)
        dd = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)        # [d, nb, 1]
        q = b[:, :, 2:].view(np.int8).astype(np.float64)
        return (dd * q).reshape(d, n)
    if name == "q4_K":
        b = W.reshape(d, n // 256, 144)
        dd = b[:, :, 0:2].copy().view(np.float16).astype(np.float64)
        dm = b[:, :, 2:4].copy().view(np.float16).astype(np.float64)
        s = b[:, :, 4:16].astype(np.int64)
        sc = np.zeros(s.shape[:2] + (8,), np.int64)
        mn = np.zeros_like(sc)
        sc[..., :4] = s[..., 0:4] & 63
        mn[..., :4] = s[..., 4:8] & 63
        sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
        mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
        q = b[:, :, 16:].reshape(d, n // 256, 4, 32).astype(np.int64)
        vals = np.concatenate([q & 15, q >> 4], axis=-1)        # [d, nb, 4, 64]
        scale = sc.reshape(d, n // 256, 4, 2)
        mins = mn.reshape(d, n // 256, 4, 2)
        s64 = np.repeat(scale, 32, axis=-1)
        m64 = np.repeat(mins, 32, axis=-1)
        w = dd[..., None] * s64 * vals - dm[..., None] * m64
        return w.reshape(d, n)
    if name == "q6_K":
        b = W.reshape(d, n // 256, 210)
        ql = b[:, :, 0:128].astype(np.int64).reshape(d, -1, 2, 64)
        qh = b[:, :, 128:192].astype(np.int64).reshape(d, -1, 2, 32)
        sc = b[:, :, 192:208].view(np.int8).astype(np.float64)
        dd = b[:, :, 208:210].copy().view(np.float16).astype(np.float64)
        vals = np.empty(ql.shape[:3] + (128,), np.int64)
        for quarter in range(4):
            lo = ql[..., 32:64] if quarter & 1 else ql[..., 0:32]
            nib = (lo >> 4) if quarter & 2 else (lo & 15)
            vals[..., 32 * quarter:32 * quarter + 32] = nib | (((qh >> (2 * quarter)) & 3) << 4)
        vals = vals.reshape(d, -1, 256) - 32
        w = dd * np.repeat(sc, 16, axis=-1) * vals
        return w.reshape(d, n)
    raise ValueError(name)


def test_known_answers(oracle_mod):
    O = oracle_mod
    one = np.float16(1.0).view(np.uint16)
    # Q8_0: d = 1, qs = -16..15, x = 1 -> sum = -16
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([one], np.uint16).view(np.uint8)
    blk[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    assert O.matmul(blk, np.ones(32, np.float32), 32, 1, O.TYPE_Q8_0)[0] == -16.0
    # Q4_K: d = 1, dmin = 0.5, every sub-block scale 1 and min 2, quant 7:
    # every weight 7 - 1 = 6, so x = 1 gives 256 * 6
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([one], np.uint16).view(np.uint8)
    blk[2:4] = np.array([np.float16(0.5).view(np.uint16)], np.uint16).view(np.uint8)
    blk[4:8] = 1          # scales of sub-blocks 0..3
    blk[8:12] = 2         # mins of sub-blocks 0..3
    blk[12:16] = 0x21     # sub-blocks 4..7: scale 1 (low nibble), min 2 (high)
    blk[16:] = 0x77
    assert O.matmul(blk, np.ones(256, np.float32), 256, 1, O.TYPE_Q4_K)[0] == 1536.0
    # Q6_K: d = 0.25, scales 4, every 6-bit value 33 (-> 1): weight 1 each
    blk = np.zeros(210, np.uint8)
    blk[0:128] = 0x11     # low nibbles 1
    blk[128:192] = 0xAA   # high bit pairs 2 -> 32 + 1 = 33
    blk[192:208] = 4
    blk[208:210] = np.array([np.float16(0.25).view(np.uint16)], np.uint16).view(np.uint8)
    x = np.arange(256, dtype=np.float32)
    assert O.matmul(blk, x, 256, 1, O.TYPE_Q6_K)[0] == float(x.sum())
    # zero scales give exact zeros whatever the quants and x
    rng = np.random.default_rng(3)
    for name in ("q4_K", "q6_K", "q8_0"):
        W = _rows(O, rng, name, 256, 4)
        if name == "q4_K":
            W.reshape(4, 144)[:, 0:4] = 0
        elif name == "q6_K":
            W.reshape(4, 210)[:, 208:210] = 0
        else:
            W.reshape(4, -1, 34)[:, :, 0:2] = 0
        out = O.matmul(W, rng.standard_normal(256).astype(np.float32), 256, 4, TYPES[name])
        assert not out.any()


def test_unsupported_type_rejected(oracle_mod):
    with pytest.raises(ValueError):
        oracle_mod.matmul(np.zeros(18, np.uint8), np.zeros(32, np.float32), 32, 1, 2)


def test_threaded_matmul_is_bit_identical(oracle_mod):
    """The CPU baseline's row-split matmul (the reference's pool split) gives
    exactly the single-thread oracle's outputs."""
    O = oracle_mod
    rng = np.random.default_rng(21)
    for name in ("q4_K", "q6_K", "q8_0"):
        n, d = 512, 37
        W = _rows(O, rng, name, n, d)
        x = rng.standard_normal(n).astype(np.float32)
        a = O.matmul(W, x, n, d, TYPES[name])
        for thr in (1, 3, 8):
            b = O.matmul_mt(W, x, n, d, TYPES[name], thr)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (name, thr)
