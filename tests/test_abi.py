"""The C ABI without a GPU: the product library loads, exports every function
declared in include/*.h, and the gpu.h-style boundary compiles both against
this package's model.h and against the reference's own (drop-in check)."""
import ctypes as C
import os
import re
import subprocess

import pytest

from conftest import ROOT

INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(ROOT, "picolm_amd", "lib", "libpicolm_hip.so")
REF_PICOLM = "/root/reference/picolm"


def declared_functions(header=None):
    names = set()
    for h in sorted(os.listdir(INCLUDE)):
        if not h.endswith(".h") or (header and h != header):
            continue
        text = open(os.path.join(INCLUDE, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        # the USE_HIP branch of gpu_hip.h declares the real functions; skip the stubs
        text = re.sub(r"#else /\* !USE_HIP \*/.*?#endif /\* USE_HIP \*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(",
                             text, flags=re.M):
            name = m.group(1)
            if name not in ("defined", "if", "sizeof"):
                names.add(name)
    return names


def exported(path):
    r = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return {line.split()[-1] for line in r.stdout.splitlines() if " T " in line}


def test_library_exports_every_device_function():
    lib = C.CDLL(LIB)
    names = declared_functions("picolm_hip.h")
    assert len(names) >= 30
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_library_exports_plh_only():
    """The kernel library carries no gpu_* symbol: gpu_hip.c reads the host
    program's model_t and is compiled inside that program against its own
    model.h, so no copy built against another layout can be linked by
    mistake."""
    syms = exported(LIB)
    assert not [s for s in syms if s.startswith("gpu_")]
    assert declared_functions("picolm_hip.h") <= syms


def test_boundary_source_defines_every_gpu_function(tmp_path):
    """Every gpu_* declared by include/gpu_hip.h is defined by gpu_hip.c."""
    obj = tmp_path / "gpu_hip.o"
    r = _gcc(["-c", "-fPIC", "-DUSE_HIP", "-I" + INCLUDE,
              "-I" + os.path.join(ROOT, "picolm_amd", "host"),
              os.path.join(ROOT, "picolm_amd", "host", "gpu_hip.c"), "-o", str(obj)])
    assert r.returncode == 0, r.stderr
    r = subprocess.run(["nm", "--defined-only", str(obj)], capture_output=True, text=True)
    defined = {line.split()[-1] for line in r.stdout.splitlines() if " T " in line}
    want = declared_functions("gpu_hip.h")
    assert len(want) >= 10 and want <= defined, sorted(want - defined)


def test_python_binding_covers_the_device_abi():
    import picolm_amd._native as N
    plh = {n for n in declared_functions() if n.startswith("plh_")}
    assert plh <= set(N._SIGS), sorted(plh - set(N._SIGS))


def test_library_fails_loudly_without_a_device():
    """No fallback: with no HIP device, init returns -1 with a message and
    every entry point refuses to run."""
    import picolm_amd as P
    if P.lib.plh_device_count() > 0:
        pytest.skip("a device is visible")
    assert P.lib.plh_init(0) == -1
    assert P.lib.plh_available() == 0
    rc = P.lib.plh_attn_decode(1, 4, 1, 64, 8, 0, 0, 1, 0, *([None] * 8))
    assert rc == -1 and "not initialised" in P._native.last_error()
    with pytest.raises(P.PicolmHipError):
        P.init(0)


def _gcc(args):
    return subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror"] + args,
                          capture_output=True, text=True)


def test_boundary_compiles_against_package_model_h():
    r = _gcc(["-fsyntax-only", "-DUSE_HIP", "-I" + INCLUDE,
              "-I" + os.path.join(ROOT, "picolm_amd", "host"),
              os.path.join(ROOT, "picolm_amd", "host", "gpu_hip.c")])
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not os.path.isdir(REF_PICOLM), reason="reference sources not present")
def test_boundary_compiles_against_reference_model_h():
    """gpu_hip.c reads only model_t fields that the reference defines with the
    same names, so it builds unchanged inside picolm."""
    r = _gcc(["-fsyntax-only", "-DUSE_HIP", "-D_GNU_SOURCE", "-I" + INCLUDE, "-I" + REF_PICOLM,
              os.path.join(ROOT, "picolm_amd", "host", "gpu_hip.c")])
    assert r.returncode == 0, r.stderr


def test_stubs_without_use_hip(tmp_path):
    """Without USE_HIP every entry point is an inline stub returning -1 / 0
    (gpu.h:31-42 convention), so call sites compile and fall back."""
    src = tmp_path / "stub.c"
    src.write_text('''
#include "gpu_hip.h"
int main(void) {
    model_t m = {0};
    float f[4] = {0};
    int bad = 0;
    bad |= gpu_init(&m) != -1;
    bad |= gpu_upload_model(&m) != -1;
    bad |= gpu_available() != 0;
    bad |= gpu_try_matmul(f, f, f, 1, 1, 0) != -1;
    bad |= gpu_try_attention(&m, 0, 0, f, f, f, f) != -1;
    bad |= gpu_try_attention_prefill(&m, 0, 0, 1, f, f, f, f) != -1;
    bad |= gpu_kv_download(&m, 1) != -1;
    bad |= gpu_kv_upload(&m, 1) != -1;
    gpu_shutdown();
    return bad;
}
''')
    exe = tmp_path / "stub"
    r = _gcc(["-I" + INCLUDE, "-I" + os.path.join(ROOT, "picolm_amd", "host"), str(src), "-o",
              str(exe)])
    assert r.returncode == 0, r.stderr
    assert subprocess.run([str(exe)]).returncode == 0


def test_set_tuning_checks_prefetch_setting():
    """plh_set_tuning needs no device: key 15 (the forward pass's L2 weight
    prefetch) takes -1, 0 and 1 and refuses anything else, and an unknown key
    is refused."""
    import picolm_amd as P
    for v in (-1, 1, 0):
        assert P.lib.plh_set_tuning(15, v) == 0
    for v in (-2, 2):
        assert P.lib.plh_set_tuning(15, v) == -1
        assert "forward weight prefetch" in P._native.last_error()
    for v in (-1, 8, 31, 0):
        assert P.lib.plh_set_tuning(17, v) == 0
    for v in (-2, 1, 7, 32):
        assert P.lib.plh_set_tuning(17, v) == -1
        assert "fusion" in P._native.last_error()
    assert P.lib.plh_set_tuning(99, 0) == -1
    assert "unknown key" in P._native.last_error()
