"""The C-ABI library: it loads, exports every symbol include/q8_rt.h declares, and its host-side
functions behave as the reference's (no GPU needed)."""
import os
import subprocess
import sys

import numpy as np
import pytest

import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_header_symbols_exported(q8rt):
    lib = q8rt.load()
    names = q8rt.header_symbols()
    assert {"rt_init", "rt_gemv", "rt_gemv_q", "rt_gemv_open", "rt_gemv_go", "rt_gemm", "rt_gemm_q", "gemv_i_bytes", "gemv_i_repack"} <= set(names)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes view binds every one of them
    assert set(names) == set(q8rt._SIGS), set(names) ^ set(q8rt._SIGS)


def test_gemv_i_bytes(q8rt):
    lib = q8rt.load()
    for rows, cols in [(16, 32), (4096, 4096), (12288, 4096), (151936, 4096)]:
        assert lib.gemv_i_bytes(rows, cols) == rows // 16 * (cols // 32) * 544 == rows * cols // 32 * 34


def test_gemv_i_repack_host(q8rt, oracle):
    lib = q8rt.load()
    for rows, cols in [(16, 32), (48, 96), (64, 512)]:
        q8, _ = synth.case(rows + cols, rows, cols, 1)
        out = np.empty_like(q8)
        lib.gemv_i_repack(q8rt.ptr(q8), rows, cols, q8rt.ptr(out))
        assert np.array_equal(out, oracle.repack_s(q8, rows, cols))


def _run(code):
    return subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=120)


def test_bad_shape_aborts_with_reason():
    """A violation of rows % 16 / cols % 32 prints the reason and aborts (no partial result)."""
    code = ("import sys; sys.path.insert(0, 'tests'); from conftest import load_package; import numpy as np; "
            "m = load_package(); lib = m.load(); a = np.zeros(1024, np.uint8); lib.gemv_i_repack(m.ptr(a), 15, 32, m.ptr(a))")
    p = _run(code)
    assert p.returncode == -6, (p.returncode, p.stderr)
    assert "gemv_i_repack" in p.stderr and "multiple of 16" in p.stderr


def test_rt_init_without_gpu():
    """rt_init returns -1 (it does not abort) where no GPU is visible."""
    code = ("import sys, ctypes; sys.path.insert(0, 'tests'); from conftest import load_package; m = load_package(); lib = m.load(); "
            "r = m.Rt(); print(lib.rt_init(ctypes.byref(r), 1))")
    p = _run(code)
    assert p.returncode == 0, p.stderr
    if p.stdout.strip() == "0":
        pytest.skip("a GPU is visible here")
    assert p.stdout.strip() == "-1"


def test_c_caller_compiles_and_links(tmp_path):
    """A C caller written against include/q8_rt.h alone (tests/c/drop_in.c) compiles with gcc and links."""
    exe = tmp_path / "drop_in"
    p = subprocess.run(["gcc", "-std=gnu11", "-O2", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "c", "drop_in.c"), "-L", os.path.join(ROOT, "intel-phi-apl_amd"), "-lq8rt",
                        "-Wl,-rpath," + os.path.join(ROOT, "intel-phi-apl_amd"), "-lm", "-o", str(exe)], capture_output=True, text=True)
    assert p.returncode == 0, p.stderr


REF_CARD = "/root/reference/src/card"


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_CARD, "rt.h")), reason="the reference's sources are not here (only in the build container)")
def test_reference_header_identical(tmp_path):
    """A caller compiled against the reference's own src/card/rt.h links against libq8rt.so with
    link-time type checking: every product entry point's parameter and return types (rt.h:38-39,
    61-72, 85) are the reference's (-Werror=lto-type-mismatch), and struct rt's size, field offsets
    and RT_BATCH (rt.h:19-26, 66) equal this library's."""
    inc, lib = os.path.join(ROOT, "include"), os.path.join(ROOT, "intel-phi-apl_amd")
    objs = []
    for src, flag in (("ref_abi_ref.c", REF_CARD), ("ref_abi_own.c", inc)):
        o = tmp_path / (src + ".o")
        p = subprocess.run(["gcc", "-std=gnu11", "-O1", "-flto", "-Wall", "-Werror", "-I", flag, "-c", os.path.join(ROOT, "tests", "c", src), "-o", str(o)],
                           capture_output=True, text=True)
        assert p.returncode == 0, p.stderr
        objs.append(str(o))
    exe = tmp_path / "ref_abi"
    p = subprocess.run(["gcc", "-O1", "-flto", "-Werror=lto-type-mismatch", *objs, "-L", lib, "-lq8rt", "-Wl,-rpath," + lib, "-o", str(exe)],
                       capture_output=True, text=True)
    assert p.returncode == 0, p.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "layout identical" in r.stdout
