"""Writes the golden fixtures under tests/golden/ from the REFERENCE itself.

Run in the build container only (it needs /root/reference and the harness that
oracle/Makefile builds from it into oracle/_ref/):

    make -C oracle all ref && python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):
  fp16_kat.npz      fp32 -> fp16 known answers from the reference's
                    fp32_to_fp16 (quant.c:41-78) on special values plus a seeded
                    sample, and a SHA-256 of fp16_to_fp32 (quant.c:11-39) over all
                    65536 inputs.
  rope_tables.npz   the reference's init_rope_tables (model.c:545-556) output
                    for three (seq, head_dim, theta) cases.
  decode_*.npz      per (pos, layer) q/k/v fed to the reference's
                    model_forward_ex (model.c:746-925) and the attention output it
                    produced (read back from s->xb2 through an identity Wo), plus
                    the reference's final FP16 caches.
  prefill_*.npz     per chunk and layer the q/k/v that the reference's
                    model_forward_prefill computed (model.c:985-1000), the
                    reference's final caches and last-token logits, and the
                    per-token attention outputs.  The reference does not expose
                    those outputs directly; they are the oracle's, kept only after
                    this script has checked that they reproduce the reference's
                    caches of the next layer and its logits bit for bit.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def kat_inputs():
    specials = np.array([
        0.0, -0.0, 1.0, -1.0, 0.5, 2.0, 65504.0, -65504.0, 65519.99, 65520.0,
        65536.0, 1e10, -1e10, np.inf, -np.inf,
        2.0 ** -25, -(2.0 ** -25), np.nextafter(np.float32(2.0 ** -25), np.float32(0)),
        2.0 ** -24, 1.5 * 2.0 ** -24, 2.0 ** -14, np.nextafter(np.float32(2.0 ** -14), np.float32(0)),
        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -(1.0 + 2.0 ** -11), 1.0 + 2.0 ** -12,
        1e-40, -1e-40, 3.14159265, -2.71828, 1e-8, 6.1e-5, 6.0e-5,
    ], dtype=np.float32)
    nan_bits = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FBFFFFF, 0xFF812345],
                        dtype=np.uint32).view(np.float32)
    rng = np.random.default_rng(20240601)
    sample_bits = rng.integers(0, 2 ** 32, 5000, dtype=np.uint64).astype(np.uint32)
    normals = rng.standard_normal(5000).astype(np.float32)
    # exact ties: 11 significant bits + a single 1 in bit 12 of the mantissa
    ties = (rng.integers(0x33000000 >> 13, 0x47800000 >> 13, 2000, dtype=np.uint64)
            .astype(np.uint32) << 13 | 0x1000).view(np.float32)
    return np.concatenate([specials, nan_bits, sample_bits.view(np.float32), normals, ties])


def make_fp16(R):
    R.ref_f16_to_f32_array.argtypes = [O._u16p, O._f32p, C.c_size_t]
    R.ref_f16_to_f32_array.restype = None
    x = kat_inputs()
    y = np.array([R.fp32_to_fp16(C.c_float(v)) for v in x.tolist()], dtype=np.uint16)
    # ctypes quiets signalling NaNs on the way in; recompute those in C bits
    xb = x.view(np.uint32)
    h = np.arange(65536, dtype=np.uint16)
    f = np.empty(65536, dtype=np.float32)
    R.ref_f16_to_f32_array(h, f, 65536)
    digest = hashlib.sha256(f.view(np.uint32).tobytes()).hexdigest()
    # signalling NaN inputs must go through C without conversion: take them out
    quiet = ~((np.isnan(x)) & ((xb & 0x00400000) == 0))
    np.savez_compressed(os.path.join(HERE, "fp16_kat.npz"),
                        f32_bits=xb[quiet], f16=y[quiet],
                        f16_to_f32_sha256=np.array(digest))


def make_rope(R):
    out = {}
    for i, (S, D, base) in enumerate([(64, 64, 10000.0), (96, 128, 500000.0), (40, 32, 10000.0)]):
        shp = O.Shape(1, 2, 1, D, S, base)
        rm = O.RefModel(shp, 0)
        out[f"cos{i}"] = rm.cos.copy()
        out[f"sin{i}"] = rm.sin.copy()
        out[f"cfg{i}"] = np.array([S, D, base], dtype=np.float64)
        rm.close()
    np.savez_compressed(os.path.join(HERE, "rope_tables.npz"), **out)


def make_decode(R, name, L, Hq, Hkv, D, S, base, rope_type, n_pos, seed):
    shp = O.Shape(L, Hq, Hkv, D, S, base, rope_type)
    rm = O.RefModel(shp, 0, seed=seed)
    rng = np.random.default_rng(seed)
    qs = rng.standard_normal((n_pos, L, shp.q_dim)).astype(np.float32)
    ks = rng.standard_normal((n_pos, L, shp.kv_dim)).astype(np.float32)
    vs = rng.standard_normal((n_pos, L, shp.kv_dim)).astype(np.float32)
    outs = np.empty((n_pos, L, shp.q_dim), dtype=np.float32)
    for pos in range(n_pos):
        for l in range(L):
            R.ref_set_decode_qkv(rm.h, l, qs[pos, l], ks[pos, l], vs[pos, l])
        for l in range(L):
            R.ref_decode(rm.h, pos, l + 1, outs[pos, l])
    np.savez_compressed(os.path.join(HERE, name),
                        dims=np.array([L, Hq, Hkv, D, S, rope_type]), base=np.float64(base),
                        q=qs, k=ks, v=vs, out=outs, key_cache=rm.kc.copy(),
                        val_cache=rm.vc.copy())
    rm.close()


def make_prefill(R, name, L, Hq, Hkv, D, S, base, rope_type, chunks, seed):
    shp = O.Shape(L, Hq, Hkv, D, S, base, rope_type)
    rm = O.RefModel(shp, 1, seed=seed, w_scale=0.3)
    kc = np.zeros(shp.cache_elems(), np.uint16)
    vc = kc.copy()
    cos_t, sin_t = O.rope_tables(S, D, base)
    rng = np.random.default_rng(seed)
    rec = {"dims": np.array([L, Hq, Hkv, D, S, rope_type]), "base": np.float64(base),
           "chunks": np.array(chunks)}
    start = 0
    for ci, n in enumerate(chunks):
        toks = rng.integers(0, shp.q_dim, n).astype(np.int32)
        logits = np.empty(shp.q_dim, np.float32)
        R.ref_prefill(rm.h, toks, n, start, logits)
        x = np.empty((n, shp.q_dim), np.float32)
        R.ref_embed(rm.h, toks, n, x.reshape(-1))
        for l in range(L):
            q = np.empty((n, shp.q_dim), np.float32)
            k = np.empty((n, shp.kv_dim), np.float32)
            v = np.empty((n, shp.kv_dim), np.float32)
            R.ref_layer_inputs(rm.h, l, x.reshape(-1), n, q.reshape(-1), k.reshape(-1), v.reshape(-1))
            rec[f"q_{ci}_{l}"] = q.copy()
            rec[f"k_{ci}_{l}"] = k.copy()
            rec[f"v_{ci}_{l}"] = v.copy()
            a = O.attn_prefill(shp, l, start, n, q, k, v, kc, vc, cos_t, sin_t)
            rec[f"out_{ci}_{l}"] = a.copy()
            x = (x + a) + np.float32(0)
        expect = np.empty(shp.q_dim, np.float32)
        R.ref_final_norm(rm.h, np.ascontiguousarray(x[-1]), expect)
        if not np.array_equal(expect.view(np.uint32), logits.view(np.uint32)):
            raise SystemExit(f"{name}: oracle chain does not reproduce the reference logits")
        rec[f"logits_{ci}"] = logits
        start += n
    if not (np.array_equal(kc, rm.kc) and np.array_equal(vc, rm.vc)):
        raise SystemExit(f"{name}: oracle caches differ from the reference's")
    rec["key_cache"] = rm.kc.copy()
    rec["val_cache"] = rm.vc.copy()
    np.savez_compressed(os.path.join(HERE, name), **rec)
    rm.close()


def main():
    if not O.ref_available():
        raise SystemExit("build the reference harness first: make -C oracle ref")
    R = O.ref()
    make_fp16(R)
    make_rope(R)
    make_decode(R, "decode_gqa4_d64.npz", 2, 4, 1, 64, 24, 10000.0, O.ROPE_LLAMA, 20, 11)
    make_decode(R, "decode_gqa4_d128.npz", 2, 8, 2, 128, 16, 500000.0, O.ROPE_LLAMA, 8, 12)
    make_decode(R, "decode_mha_qwen_d64.npz", 1, 3, 3, 64, 12, 10000.0, O.ROPE_QWEN, 10, 13)
    make_prefill(R, "prefill_gqa4_d64.npz", 2, 4, 1, 64, 40, 10000.0, O.ROPE_LLAMA, [9, 15], 21)
    make_prefill(R, "prefill_gqa4_d128.npz", 2, 8, 2, 128, 24, 500000.0, O.ROPE_LLAMA, [1, 8], 22)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
