"""Synthetic picolm models: random GGUF weight blocks with the reference's
in-file layout (quant.h:66-125), for benches and tests where no checkpoint
can be downloaded.

Scales are chosen so that a projection of a unit-RMS vector has outputs of
order one (a 22-layer stack neither blows up nor vanishes), which keeps the
attention softmax and silu in their interesting ranges.
"""
from __future__ import annotations

import math

import numpy as np

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 2, 8, 12, 14
BLOCK = {TYPE_F32: (1, 4), TYPE_F16: (1, 2), TYPE_Q4_0: (32, 18), TYPE_Q8_0: (32, 34),
         TYPE_Q4_K: (256, 144), TYPE_Q6_K: (256, 210)}   # (weights, bytes) per block
# RMS of a dequantized weight over its fp16 super-block scale when every
# quant byte is uniform (Q4_K: scale 0..63 times quant 0..15 less the min
# term; Q6_K: int8 scale times (q - 32); Q8_0: int8 quant; Q4_0: q - 8)
_RMS_OVER_SCALE = {TYPE_Q4_K: 300.0, TYPE_Q6_K: 1365.0, TYPE_Q8_0: 74.0, TYPE_Q4_0: 4.6}

LAYER_MATRICES = ("q", "k", "v", "o", "gate", "up", "down")


def row_bytes(qtype: int, n: int) -> int:
    w, b = BLOCK[qtype]
    if n % w:
        raise ValueError(f"row of {n} weights is not whole blocks of type {qtype}")
    return n // w * b


def unit_scale_exp(qtype: int, n: int) -> tuple[float, float]:
    """Exponent range of the fp16 scales that gives W @ x outputs of RMS ~1
    for a unit-RMS x of length n."""
    c = -math.log2(math.sqrt(n) * _RMS_OVER_SCALE[qtype])
    return (c - 1.0, c + 1.0)


def random_weights(rng: np.random.Generator, qtype: int, n: int, d: int,
                   scale_exp=(-12, -4)) -> np.ndarray:
    """d rows of random blocks of a GGUF type: every quant byte uniform, the
    fp16 scales finite with exponents in scale_exp (2^lo .. 2^hi magnitude),
    Q6_K's int8 scales uniform.  F32 / F16 rows are standard normal.
    Returns uint8 [d, row_bytes]."""
    rb = row_bytes(qtype, n)
    if qtype == TYPE_F32:
        W = rng.standard_normal((d, n), dtype=np.float32).view(np.uint8).reshape(d, rb)
        return np.ascontiguousarray(W)
    if qtype == TYPE_F16:
        return np.ascontiguousarray(
            rng.standard_normal((d, n)).astype(np.float16).view(np.uint8).reshape(d, rb))
    W = rng.integers(0, 256, size=(d, rb), dtype=np.uint8)
    nb = n // BLOCK[qtype][0]
    blocks = W.reshape(d, nb, BLOCK[qtype][1])

    def f16_field(shape):
        mag = np.exp2(rng.uniform(*scale_exp, size=shape)).astype(np.float16)
        signed = qtype in (TYPE_Q8_0, TYPE_Q6_K, TYPE_Q4_0)
        sign = rng.choice(np.array([-1, 1], np.float16), size=shape) if signed else np.float16(1)
        return (mag * sign).astype(np.float16).view(np.uint16)

    def put(lo, shape):
        blocks[:, :, lo:lo + 2] = f16_field(shape).view(np.uint8).reshape(d, nb, 2)
    if qtype == TYPE_Q4_K:
        put(0, (d, nb))
        put(2, (d, nb))
    elif qtype == TYPE_Q6_K:
        put(208, (d, nb))
    elif qtype in (TYPE_Q8_0, TYPE_Q4_0):
        put(0, (d, nb))
    return np.ascontiguousarray(W)


class SynthModel:
    """Host buffers of a LLaMA / Qwen-shaped model in picolm's terms.

    Attributes: the config ints (n_layers, n_embd, n_ffn, n_heads,
    n_kv_heads, head_dim, vocab_size, max_seq_len, rope_type), rope_base,
    eps; embd_type + token_embd (uint8 [vocab, row_bytes]); output_norm
    (fp32); output_type + output; layers: list of dicts with attn_norm,
    ffn_norm (fp32), q, k, v, o, gate, up, down as (qtype, uint8 rows),
    q_bias, k_bias, v_bias, o_bias, q_norm, k_norm (fp32 or None).

    types: GGUF type per role ("embd", "output", and the layer matrices);
    a per-layer list is allowed for layer matrices.  share_layers reuses one
    random layer's bytes for every layer (host memory and generation time;
    each layer still gets its own device copy).
    """

    DEFAULT_TYPES = dict(embd=TYPE_Q4_K, output=TYPE_Q6_K, q=TYPE_Q4_K, k=TYPE_Q4_K,
                         v=TYPE_Q6_K, o=TYPE_Q4_K, gate=TYPE_Q4_K, up=TYPE_Q4_K, down=TYPE_Q6_K)

    def __init__(self, n_layers, n_embd, n_ffn, n_heads, n_kv_heads, head_dim, vocab_size,
                 max_seq_len, rope_type=0, rope_base=1e4, eps=1e-5, types=None, seed=0,
                 biases=False, qk_norm=False, share_layers=False):
        self.n_layers, self.n_embd, self.n_ffn = n_layers, n_embd, n_ffn
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, head_dim
        self.vocab_size, self.max_seq_len = vocab_size, max_seq_len
        self.rope_type, self.rope_base, self.eps = rope_type, float(rope_base), float(eps)
        t = dict(self.DEFAULT_TYPES)
        t.update(types or {})
        self.types = t
        rng = np.random.default_rng(seed)
        q_dim, kv_dim = n_heads * head_dim, n_kv_heads * head_dim

        def mat(qtype, n, d):
            if qtype in (TYPE_F32, TYPE_F16):
                W = random_weights(rng, qtype, n, d)
                if qtype == TYPE_F32:   # N(0, 1/n): unit-RMS outputs
                    W = (W.view(np.float32) / np.float32(math.sqrt(n))).view(np.uint8)
                return np.ascontiguousarray(W)
            return random_weights(rng, qtype, n, d, unit_scale_exp(qtype, n))

        def norm(n):
            return rng.uniform(0.5, 1.5, n).astype(np.float32)

        self.embd_type = t["embd"]
        self.token_embd = mat(self.embd_type, n_embd, vocab_size)
        self.output_norm = norm(n_embd)
        self.output_type = t["output"]
        self.output = mat(self.output_type, n_embd, vocab_size)
        shapes = dict(q=(n_embd, q_dim), k=(n_embd, kv_dim), v=(n_embd, kv_dim),
                      o=(q_dim, n_embd), gate=(n_embd, n_ffn), up=(n_embd, n_ffn),
                      down=(n_ffn, n_embd))
        self.layers = []
        for li in range(n_layers):
            if share_layers and li > 0:
                self.layers.append(self.layers[0])
                continue
            L = dict(attn_norm=norm(n_embd), ffn_norm=norm(n_embd))
            for name in LAYER_MATRICES:
                qt = t[name][li] if isinstance(t[name], (list, tuple)) else t[name]
                L[name] = (qt, mat(qt, *shapes[name]))
            def vec(n, on):
                return (rng.standard_normal(n) * 0.1).astype(np.float32) if on else None
            L["q_bias"], L["k_bias"] = vec(q_dim, biases), vec(kv_dim, biases)
            L["v_bias"], L["o_bias"] = vec(kv_dim, biases), vec(n_embd, biases)
            L["q_norm"] = norm(head_dim) if qk_norm else None
            L["k_norm"] = norm(head_dim) if qk_norm else None
            self.layers.append(L)

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    def cache_elems(self) -> int:
        return self.n_layers * self.max_seq_len * self.kv_dim

    def weight_bytes_per_token(self) -> int:
        """GGUF bytes of every matrix one decode token streams (projections
        of all layers and the output matrix; the embedding reads one row)."""
        total = self.output.nbytes + self.token_embd.nbytes // self.vocab_size
        for L in self.layers:
            total += sum(L[name][1].nbytes for name in LAYER_MATRICES)
        return total
