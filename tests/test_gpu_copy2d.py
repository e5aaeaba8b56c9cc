"""plh_copy2d_batch_async, the one-launch copy that brings a forward pass's
x and appended cache rows back into pinned host memory (gpu_try_forward's
copy-back, standing in for model.c's in-place writes of state.x and the
cache rows, model.c:822-826): every byte of each strided copy lands where
numpy's own slicing puts it, bytes outside the copies stay untouched, for the
16-byte, 4-byte and 1-byte unit paths, into device and pinned host memory."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class Copy2D(C.Structure):
    _fields_ = [("dst", C.c_void_p), ("dpitch", C.c_size_t), ("src", C.c_void_p),
                ("spitch", C.c_size_t), ("width", C.c_size_t), ("height", C.c_size_t)]


def host_bytes(ptr, n):
    return np.ctypeslib.as_array((C.c_uint8 * n).from_address(ptr))


# (dst offset, dpitch, src offset, spitch, width, height) per copy
CASES = {
    # gpu_try_forward's shape: x, then 22 layers' key and value rows
    "forward_copy_back": [(0, 8192, 0, 8192, 8192, 1),
                          (8192, 512, 8192, 4096, 512, 22),
                          (8192 + 11264, 512, 8192 + 22 * 4096, 4096, 512, 22)],
    "dword_units": [(4, 36, 8, 44, 36, 7), (400, 12, 1000, 100, 12, 30)],
    "byte_units": [(3, 21, 5, 33, 17, 9)],
    "one_big_copy": [(0, 96 * 1024, 16, 128 * 1024, 96 * 1024, 40)],
    "empty_copies_skipped": [(0, 64, 0, 64, 0, 5), (64, 64, 64, 128, 64, 3),
                             (0, 64, 0, 64, 64, 0), (512, 32, 1024, 48, 32, 4)],
}


def span(off, pitch, width, height):
    return off + (pitch * (height - 1) + width if height and width else 0)


@pytest.mark.parametrize("to_host", [True, False], ids=["pinned_host", "device"])
@pytest.mark.parametrize("name", list(CASES))
def test_copy2d_batch_matches_numpy(gpu, name, to_host):
    copies = CASES[name]
    src_n = max(span(so, sp, w, h) for _, _, so, sp, w, h in copies) + 64
    dst_n = max(span(do, dp, w, h) for do, dp, _, _, w, h in copies) + 64
    rng = np.random.default_rng(len(name))
    src = rng.integers(0, 256, src_n, dtype=np.uint8)
    fill = rng.integers(0, 256, dst_n, dtype=np.uint8)
    dsrc = gpu.DeviceBuffer.from_numpy(src)
    if to_host:
        hp = gpu.lib.plh_host_alloc(dst_n)
        assert hp
        host_bytes(hp, dst_n)[:] = fill
        dst_ptr = hp
    else:
        ddst = gpu.DeviceBuffer.from_numpy(fill)
        dst_ptr = ddst.ptr
    arr = (Copy2D * len(copies))(*[Copy2D(dst_ptr + do, dp, dsrc.ptr + so, sp, w, h)
                                  for do, dp, so, sp, w, h in copies])
    want = fill.copy()
    for do, dp, so, sp, w, h in copies:
        for r in range(h):
            want[do + r * dp:do + r * dp + w] = src[so + r * sp:so + r * sp + w]
    # twice in a row: the second call must give the same bytes
    for _ in range(2):
        gpu.check(gpu.lib.plh_copy2d_batch_async(arr, len(copies)), "plh_copy2d_batch_async")
        gpu.synchronize()
        got = host_bytes(dst_ptr, dst_n).copy() if to_host else ddst.download(np.uint8, (dst_n,))
        np.testing.assert_array_equal(got, want)
    if to_host:
        gpu.check(gpu.lib.plh_host_free(hp), "plh_host_free")


def test_copy2d_batch_rejects_bad_arguments(gpu):
    d = gpu.DeviceBuffer(4096)
    ok = Copy2D(d.ptr, 64, d.ptr + 2048, 64, 64, 2)
    assert gpu.lib.plh_copy2d_batch_async((Copy2D * 1)(ok), 0) == -1
    assert gpu.lib.plh_copy2d_batch_async((Copy2D * 5)(*[ok] * 5), 5) == -1
    assert gpu.lib.plh_copy2d_batch_async(None, 1) == -1
    null_src = Copy2D(d.ptr, 64, None, 64, 64, 2)
    assert gpu.lib.plh_copy2d_batch_async((Copy2D * 1)(null_src), 1) == -1
    assert b"null" in gpu.lib.plh_last_error()
    short_pitch = Copy2D(d.ptr, 32, d.ptr + 2048, 64, 64, 2)
    assert gpu.lib.plh_copy2d_batch_async((Copy2D * 1)(short_pitch), 1) == -1
    assert b"pitch" in gpu.lib.plh_last_error()
    gpu.synchronize()
