"""The matrix-core decode kernel (gemv_mx, 3 and 4 tokens) at every instantiated wave count (K = 2048,
4096, 6144, 8192, 12288, 16384) and row-group count (1, 2, 4, forced through Q8_GEMV_MX): the
product, the fused pair and the residual against the F64 closed form at the parity bar of
tests/parity.py, the residual bit for bit against the product plus one F32 add (in place too), and
tokens past t never read (x rows past t hold NaN). Q8_GEMV_MX = 0 checks that the VALU kernel takes
the same calls and meets the same bar."""
import ctypes as c
import os

import numpy as np
import pytest

import synth
from parity import assert_parity
from test_gpu_parity import Dev

pytestmark = pytest.mark.gpu

KS = [2048, 4096, 6144, 8192, 12288, 16384]


def say(*a):
    print(*a, flush=True)


def _run(rt, rows, cols, t, rg, seed):
    rng = np.random.default_rng(seed)
    q8g = synth.q8_rows(rng, rows, cols, "lognormal")
    q8u = synth.q8_rows(rng, rows, cols)
    x = synth.x_f32(rng, t, cols)
    xp = np.full((4, cols), np.nan, np.float32)  # rows past t: NaN, never read
    xp[:t] = x
    r = rng.standard_normal((t, rows)).astype(np.float32)
    old = os.environ.get("Q8_GEMV_MX")
    os.environ["Q8_GEMV_MX"] = rg
    wg, wu = rt.upload(q8g, rows, cols), rt.upload(q8u, rows, cols)
    try:
        with Dev(rt) as d:
            dx, dy, dp, dr, dz = d.put(xp), d.empty(4 * t * rows), d.empty(4 * t * rows), d.put(r), d.empty(4 * t * rows)
            rt.lib.rt_gemm_dev(rt.R, c.c_void_p(wg), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dy))
            rt.lib.rt_gemv_swiglu_dev(rt.R, c.c_void_p(wg), c.c_void_p(wu), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dp))
            rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(wg), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dr), c.c_void_p(dz))
            rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(wg), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dr), c.c_void_p(dr))
            y, p, z, zin = (d.get(b, (t, rows), np.float32) for b in (dy, dp, dz, dr))
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(wg))
        rt.lib.rt_q8_free(rt.R, c.c_void_p(wu))
        if old is None:
            os.environ.pop("Q8_GEMV_MX", None)
        else:
            os.environ["Q8_GEMV_MX"] = old
    return q8g, q8u, x, r, y, p, z, zin


@pytest.mark.parametrize("rg", ["1", "2", "4", "0"])
@pytest.mark.parametrize("cols", KS)
@pytest.mark.parametrize("t", [3, 4])
def test_matrix_core_decode(rt, oracle, cols, t, rg):
    rows = 64
    say(f"gemv_mx {rows}x{cols} t={t} row groups {rg}")
    q8g, q8u, x, r, y, p, z, zin = _run(rt, rows, cols, t, rg, 31 * cols + 7 * t + int(rg))
    yg = oracle.gemm_f64(q8g, rows, cols, x)
    assert_parity(y, yg, f"product {rows}x{cols} t={t} rg={rg}")
    assert_parity(p, oracle.swiglu_f64(yg, oracle.gemm_f64(q8u, rows, cols, x)), f"pair {rows}x{cols} t={t} rg={rg}")
    assert np.array_equal(z.view(np.uint32), (r + y).view(np.uint32))
    assert np.array_equal(zin.view(np.uint32), z.view(np.uint32))


def test_matrix_core_decode_tall(rt, oracle):
    """A tall matrix whose row groups the default chooser splits 4 a workgroup, odd row count of
    workgroups: 9232 rows (2308 groups, 577 workgroups) x 4096 at 4 tokens."""
    rows, cols, t = 9232, 4096, 4
    say(f"gemv_mx {rows}x{cols} t={t}")
    q8g, q8u, x, r, y, p, z, zin = _run(rt, rows, cols, t, "4", 99)
    yg = oracle.gemm_f64(q8g, rows, cols, x)
    assert_parity(y, yg, "tall product")
    assert_parity(p, oracle.swiglu_f64(yg, oracle.gemm_f64(q8u, rows, cols, x)), "tall pair")
    assert np.array_equal(z.view(np.uint32), (r + y).view(np.uint32))


def test_matrix_core_decode_in_a_graph(rt):
    """The kernel's products recorded into a graph (the product at 4 tokens, the pair at 3, the
    residual in place at 4) and replayed three times with eager work between: every replay's bits
    equal the eager run's."""
    rows, cols = 128, 4096
    rng = np.random.default_rng(5)
    mats = [synth.q8_rows(rng, rows, cols) for _ in range(3)]
    x = synth.x_f32(rng, 4, cols)
    r = rng.standard_normal((4, rows)).astype(np.float32)
    old = os.environ.get("Q8_GEMV_MX")
    os.environ["Q8_GEMV_MX"] = "2"
    ws = [rt.upload(m, rows, cols) for m in mats]
    try:
        with Dev(rt) as d:
            dx, dr0, dr = d.put(x), d.put(r), d.empty(4 * 4 * rows)
            y1, y2 = d.empty(4 * 4 * rows), d.empty(4 * 3 * rows)

            def seq():
                rt.lib.rt_gemm_dev(rt.R, c.c_void_p(ws[0]), rows, cols, c.c_void_p(dx), cols, 4, c.c_void_p(y1))
                rt.lib.rt_gemv_swiglu_dev(rt.R, c.c_void_p(ws[1]), c.c_void_p(ws[2]), rows, cols, c.c_void_p(dx), cols, 3, c.c_void_p(y2))
                rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(ws[2]), rows, cols, c.c_void_p(dx), cols, 4, c.c_void_p(dr), c.c_void_p(dr))

            outs = ((y1, (4, rows)), (y2, (3, rows)), (dr, (4, rows)))
            rt.lib.rt_dev_copy(rt.R, c.c_void_p(dr), c.c_void_p(dr0), 4 * 4 * rows)
            seq()
            want = [d.get(p, s, np.float32) for p, s in outs]
            rt.lib.rt_dev_copy(rt.R, c.c_void_p(dr), c.c_void_p(dr0), 4 * 4 * rows)
            rt.lib.rt_graph_begin(rt.R)
            seq()
            g = rt.lib.rt_graph_end(rt.R)
            try:
                for rep in range(3):
                    rt.lib.rt_dev_copy(rt.R, c.c_void_p(dr), c.c_void_p(dr0), 4 * 4 * rows)
                    rt.to_dev(y1, np.zeros((4, rows), np.float32))
                    rt.lib.rt_graph_launch(rt.R, c.c_void_p(g))
                    got = [d.get(p, s, np.float32) for p, s in outs]
                    for a, b in zip(got, want):
                        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"replay {rep}"
                    seq()  # eager work between the replays
                    rt.sync()
            finally:
                rt.lib.rt_graph_free(rt.R, c.c_void_p(g))
    finally:
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
        if old is None:
            os.environ.pop("Q8_GEMV_MX", None)
        else:
            os.environ["Q8_GEMV_MX"] = old
