"""The GEMV's device layout, checked on the CPU: plh_gemv_pack_host (the
packing plh_gemv_upload performs) followed by a numpy decoding that uses the
kernel's own addressing must give back every quant, scale and min of the
reference's GGUF blocks (quant.h:66-125), for every type and a few shapes."""
import numpy as np
import pytest

import picolm_amd as P
from picolm_amd import gemv as G
from picolm_amd import synth as S

ALIGN = 256


def _planes(qtype, n, d):
    nb = n // G.BLOCK[qtype][0]
    blocks = d * nb
    up = lambda v: (v + ALIGN - 1) // ALIGN * ALIGN  # noqa: E731
    if qtype == G.TYPE_Q4_K:   # header plane, then two 16-byte quant planes
        q0 = up(blocks * 16)
        q1 = q0 + up(blocks * 64)
        return nb, (q0, q1), None, None, q1 + up(blocks * 64)
    if qtype == G.TYPE_Q6_K:
        plane = up(blocks * 16 * 4)
        scales_off = 3 * plane
        d_off = up(scales_off + blocks * 16)
        return nb, plane, scales_off, d_off, up(d_off + blocks * 2)
    plane = up(blocks * 16)
    d_off = 2 * plane
    return nb, plane, None, d_off, up(d_off + blocks * 2)


def _q6_values(blk):
    """[256] 6-bit values of one reference Q6_K block (quant.c:199-213)."""
    ql = blk[0:128].astype(np.int64).reshape(2, 64)
    qh = blk[128:192].astype(np.int64).reshape(2, 32)
    v = np.empty((2, 128), np.int64)
    for quarter in range(4):
        lo = ql[:, 32:64] if quarter & 1 else ql[:, 0:32]
        nib = (lo >> 4) if quarter & 2 else (lo & 15)
        v[:, 32 * quarter:32 * quarter + 32] = nib | (((qh >> (2 * quarter)) & 3) << 4)
    return v.reshape(256)


@pytest.mark.parametrize("qtype,n,d", [(G.TYPE_Q4_K, 512, 5), (G.TYPE_Q4_K, 2048, 3),
                                       (G.TYPE_Q6_K, 256, 7), (G.TYPE_Q6_K, 1024, 2),
                                       (G.TYPE_Q8_0, 96, 9), (G.TYPE_Q8_0, 2048, 2)])
def test_pack_roundtrip(oracle_mod, qtype, n, d):
    rng = np.random.default_rng(n + d)
    W = S.random_weights(rng, qtype, n, d)
    packed = G.pack_host(qtype, n, d, W)
    nb, plane, scales_off, d_off, total = _planes(qtype, n, d)
    assert packed.size == total == P.lib.plh_gemv_packed_bytes(qtype, n, d)
    rb = G.row_bytes(qtype, n)
    for r in range(d):
        for i in range(nb):
            b = r * nb + i
            src = W[r, i * G.BLOCK[qtype][1]:(i + 1) * G.BLOCK[qtype][1]]
            if qtype == G.TYPE_Q4_K:
                q0, q1 = plane
                assert np.array_equal(packed[16 * b:16 * b + 16], src[:16])
                for j in range(4):
                    s = 4 * b + j      # sub-block in the matrix
                    assert np.array_equal(packed[q0 + 16 * s:q0 + 16 * s + 16],
                                          src[16 + 32 * j:32 + 32 * j])
                    assert np.array_equal(packed[q1 + 16 * s:q1 + 16 * s + 16],
                                          src[32 + 32 * j:48 + 32 * j])
            elif qtype == G.TYPE_Q6_K:
                vals = _q6_values(src)
                for j in range(16):
                    g = b * 16 + j
                    L0, L1, H = (int.from_bytes(packed[p * plane + 4 * g:p * plane + 4 * g + 4]
                                                .tobytes(), "little") for p in range(3))
                    m4, m2 = 0x0F0F0F0F, 0x03030303
                    words = [(L0 & m4) | ((H & m2) << 4),
                             ((L0 >> 4) & m4) | (((H >> 2) & m2) << 4),
                             (L1 & m4) | (((H >> 4) & m2) << 4),
                             ((L1 >> 4) & m4) | (((H >> 6) & m2) << 4)]
                    dec = [(words[e // 4] >> (8 * (e % 4))) & 0xFF for e in range(16)]
                    assert dec == list(vals[16 * j:16 * j + 16]), (r, i, j)
                assert np.array_equal(packed[scales_off + 16 * b:scales_off + 16 * b + 16],
                                      src[192:208])
                assert np.array_equal(packed[d_off + 2 * b:d_off + 2 * b + 2], src[208:210])
            else:
                assert np.array_equal(packed[16 * b:16 * b + 16], src[2:18])
                assert np.array_equal(packed[plane + 16 * b:plane + 16 * b + 16], src[18:34])
                assert np.array_equal(packed[d_off + 2 * b:d_off + 2 * b + 2], src[0:2])
    assert rb * d == W.size


def test_pack_rejects_unsupported():
    with pytest.raises(ValueError):
        G.pack_host(2, 32, 1, np.zeros(18, np.uint8))           # Q4_0: no kernel
    assert P.lib.plh_gemv_packed_bytes(G.TYPE_Q4_K, 100, 1) == 0  # not whole blocks
    assert P.lib.plh_gemv_packed_bytes(G.TYPE_Q8_0, 32, 0) == 0
