"""The boundary refuses what would make a kernel read outside its matrix.

  - a `w` that is not a registered handle (a host pointer, as an engine still on the reference's own
    repack would pass; a device buffer that was never a matrix; an address inside a matrix; a freed
    handle) stops the process with the reason on stderr before anything is launched. The child
    process runs with Q8_ABORT_EXIT set, so it ends with that exit code instead of SIGABRT;
  - rt_q8_rows_dev's indices are device data: one outside the matrix gives a row of NaN and reads
    nothing, the others their rows.
"""
import ctypes as c
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = textwrap.dedent(
    """
    import ctypes as c, importlib.util, os, sys
    import numpy as np
    spec = importlib.util.spec_from_file_location("q8rt", os.path.join({root!r}, "intel-phi-apl_amd", "__init__.py"))
    q8rt = importlib.util.module_from_spec(spec); spec.loader.exec_module(q8rt)
    rt = q8rt.Runtime()
    rows, cols = 64, 256
    q8 = np.zeros(rows * cols // 32 * 34, np.uint8)
    w = rt.upload(q8, rows, cols)
    x = np.ones(cols, np.float32); y = np.zeros(rows, np.float32)
    rt.gemv(w, rows, cols, x, y)  # a registered handle: fine
    case = sys.argv[1]
    print("child: calling with", case, flush=True)
    if case == "host":
        rt.gemv(q8.ctypes.data, rows, cols, x, y)
    elif case == "device":
        p = rt.alloc(q8.nbytes)
        dx, dy = rt.alloc(4 * cols), rt.alloc(4 * rows)
        rt.lib.rt_gemm_dev(rt.R, c.c_void_p(p), rows, cols, c.c_void_p(dx), cols, 1, c.c_void_p(dy))
    elif case == "inside":
        rt.gemv(w + 17 * cols, rows - 16, cols, x, y)
    elif case == "freed":
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
        rt.gemv_q(w, rows, cols, x, y)
    elif case in ("sub_freed", "sub_live"):
        # a matrix repacked into a buffer inside a larger allocation, at an offset
        blk, src = rt.alloc(4 * q8.nbytes), rt.alloc(q8.nbytes)
        rt.to_dev(src, q8)
        sub = blk + 4096
        rt.lib.rt_q8_repack_dev(rt.R, c.c_void_p(src), rows, cols, c.c_void_p(sub))
        dx, dy = rt.alloc(4 * cols), rt.alloc(4 * rows)
        rt.lib.rt_gemm_dev(rt.R, c.c_void_p(sub), rows, cols, c.c_void_p(dx), cols, 1, c.c_void_p(dy))  # a handle: fine
        rt.sync()
        if case == "sub_freed":
            rt.free(blk)  # the allocation goes, and with it the handle inside it
        print("child: calling with", case, flush=True)
        rt.lib.rt_gemm_dev(rt.R, c.c_void_p(sub), rows, cols, c.c_void_p(dx), cols, 1, c.c_void_p(dy))
        rt.sync()
        if case == "sub_live":
            print("child: live sub-buffer handle works", flush=True)
            rt.lib.rt_q8_repack_dev(rt.R, c.c_void_p(src), rows, cols, c.c_void_p(w + 4096))
    print("child: returned", flush=True)
    """
)


@pytest.mark.parametrize("case", ["host", "device", "inside", "freed", "sub_freed", "sub_live"])
def test_unregistered_w_stops_before_launch(case):
    """sub_freed: a buffer rt_q8_repack_dev registered at an offset inside an allocation stops being a
    handle when rt_dev_free frees the allocation. sub_live: while the allocation lives it is a handle,
    and a repack into a matrix the library allocated (at an address inside it) is refused."""
    env = dict(os.environ, Q8_ABORT_EXIT="42")
    r = subprocess.run([sys.executable, "-c", CHILD.format(root=ROOT), case], env=env, capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 42, (r.returncode, r.stderr)
    assert "child: calling with" in r.stdout and "child: returned" not in r.stdout
    if case == "sub_live":
        assert "child: live sub-buffer handle works" in r.stdout
        assert "out_dev lies in a weight handle the library allocated" in r.stderr
    else:
        assert "is not a weight handle" in r.stderr


def test_row_gather_bounds(rt, oracle):
    """rt_q8_rows_dev with indices inside and outside [0, rows): the rows, and NaN rows."""
    rows, cols = 48, 512
    q8, _ = synth.case(77, rows, cols, 1)
    w = rt.upload(q8, rows, cols)
    idx = np.array([0, 47, 48, -1, 1 << 40, 5], np.int64)
    try:
        di, dz = rt.alloc(idx.nbytes), rt.alloc(4 * len(idx) * cols)
        rt.to_dev(di, idx)
        rt.lib.rt_q8_rows_dev(rt.R, c.c_void_p(w), cols, c.c_void_p(di), len(idx), c.c_void_p(dz))
        z = np.empty((len(idx), cols), np.float32)
        rt.from_dev(z, dz)
        rt.free(di)
        rt.free(dz)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    for i, r in enumerate(idx):
        if 0 <= r < rows:
            assert np.array_equal(z[i].view(np.uint32), oracle.row(q8, cols, int(r)).view(np.uint32))
        else:
            assert np.isnan(z[i]).all(), (i, r)
