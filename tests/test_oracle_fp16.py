"""Pins the oracle's fp16 conversions (quant.c:11-78).

Checks: the reference's own known answers (tests/golden/fp16_kat.npz, written
from the compiled reference by tests/golden/make_golden.py), textbook special
cases, and -- where the reference harness is built -- an exhaustive sweep of
all 2^32 fp32 inputs against the reference's fp32_to_fp16.
"""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest

from conftest import GOLDEN, needs_ref


def test_kat_vectors(oracle_mod):
    z = np.load(os.path.join(GOLDEN, "fp16_kat.npz"))
    got = oracle_mod.f32_to_f16(z["f32_bits"].view(np.float32))
    bad = np.nonzero(got != z["f16"])[0]
    assert bad.size == 0, [(hex(z["f32_bits"][i]), hex(z["f16"][i]), hex(got[i])) for i in bad[:5]]


def test_f16_to_f32_all_inputs_digest(oracle_mod):
    z = np.load(os.path.join(GOLDEN, "fp16_kat.npz"))
    f = oracle_mod.f16_to_f32(np.arange(65536, dtype=np.uint16))
    assert hashlib.sha256(f.view(np.uint32).tobytes()).hexdigest() == str(z["f16_to_f32_sha256"])


@pytest.mark.parametrize("x,h", [
    (0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (-2.0, 0xC000),
    (65504.0, 0x7BFF), (65520.0, 0x7C00), (1e10, 0x7C00), (float("inf"), 0x7C00),
    (float("-inf"), 0xFC00), (float("nan"), 0x7E00),
    (2.0 ** -24, 0x0001), (2.0 ** -25, 0x0001), (2.0 ** -14, 0x0400),
    (1e-40, 0x0000),                       # fp32 subnormal flushes to zero
    (1.0 + 2.0 ** -11, 0x3C01),            # tie: half away from zero (RNE would give 0x3C00)
    (1.0 + 3 * 2.0 ** -11, 0x3C02),        # tie on an odd LSB rounds up in both modes
    (-(1.0 + 2.0 ** -11), 0xBC01),
])
def test_known_answers(oracle_mod, x, h):
    assert oracle_mod.lib().orc_f32_to_f16(x) == h


def test_below_half_min_subnormal_flushes(oracle_mod):
    just_below = np.nextafter(np.float32(2.0 ** -25), np.float32(0))
    assert oracle_mod.f32_to_f16(np.array([just_below]))[0] == 0


def test_roundtrip_is_identity_on_fp16_values(oracle_mod):
    h = np.arange(65536, dtype=np.uint16)
    f = oracle_mod.f16_to_f32(h)
    finite = np.isfinite(f)
    back = oracle_mod.f32_to_f16(f[finite])
    # fp16 subnormals widen to fp32 normals and come back exactly; +-0 too
    assert np.array_equal(back, h[finite])


def test_conversion_monotone_on_positive_normals(oracle_mod):
    rng = np.random.default_rng(3)
    x = np.sort(np.abs(rng.standard_normal(200000)).astype(np.float32) * 100)
    h = oracle_mod.f32_to_f16(x)
    assert np.all(np.diff(h.astype(np.int64)) >= 0)


@needs_ref
def test_exhaustive_against_reference(oracle_mod):
    R = oracle_mod.ref()
    R.ref_f16_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_void_p, C.c_int,
                                     C.POINTER(C.c_uint32)]
    R.ref_f16_mismatches.restype = C.c_uint64
    fp = C.cast(oracle_mod.lib().orc_f32_to_f16, C.c_void_p)
    first_bad = C.c_uint32()
    n = R.ref_f16_mismatches(0, 1 << 32, fp, min(8, os.cpu_count() or 1), C.byref(first_bad))
    assert n == 0, hex(first_bad.value)


def test_checksum_matches_elementwise(oracle_mod):
    """orc_f16_checksum (used against the GPU's exhaustive sweep) is the
    documented sum over the range, cross-checked in numpy on a slice."""
    first, count = 0x3F800000 - 5000, 20000
    bits = np.arange(first, first + count, dtype=np.uint64)
    h = oracle_mod.f32_to_f16(bits.astype(np.uint32).view(np.float32)).astype(np.uint64)
    x = bits.copy()
    with np.errstate(over="ignore"):
        x ^= x >> np.uint64(30); x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27); x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
        want = int(np.sum((h + np.uint64(1)) * (x | np.uint64(1)), dtype=np.uint64))
    assert oracle_mod.lib().orc_f16_checksum(first, count, 3) == want
