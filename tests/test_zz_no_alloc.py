"""rt_gemm_dev_noalloc (the product that allocates nothing: its matrix-core partials live in the
library's static device scratch) against rt_gemm_dev, bit for bit, on calls in a row, each smaller
than the one before, so that every call runs over what the previous left in the scratch: the
matrix-core product with a K split (the scratch in use), without one, and the decode kernel."""
import ctypes as c

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def _product(rt, fn, w, rows, cols, x):
    t = x.shape[0]
    dx, dy = rt.alloc(x.nbytes), rt.alloc(4 * t * rows)
    try:
        rt.to_dev(dx, x)
        # NaN in y first: every output must be written by the call
        rt.to_dev(dy, np.full((t, rows), np.nan, np.float32))
        fn(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dy))
        y = np.empty((t, rows), np.float32)
        rt.from_dev(y, dy)
    finally:
        rt.free(dx)
        rt.free(dy)
    return y


def test_noalloc_equals_gemm_dev(rt):
    cases = [(12288, 4096, 40), (4096, 12288, 16), (2048, 4096, 7), (1024, 1024, 3)]
    rng = np.random.default_rng(707)
    for rows, cols, t in cases:
        q8 = synth.q8_rows(rng, rows, cols)
        x = synth.x_f32(rng, t, cols)
        w = rt.upload(q8, rows, cols)
        try:
            print(f"noalloc {rows}x{cols} t={t}", flush=True)
            got = _product(rt, rt.lib.rt_gemm_dev_noalloc, w, rows, cols, x)
            want = _product(rt, rt.lib.rt_gemm_dev, w, rows, cols, x)
            again = _product(rt, rt.lib.rt_gemm_dev_noalloc, w, rows, cols, x)
        finally:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
        assert np.all(np.isfinite(got))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (rows, cols, t)
        assert np.array_equal(again.view(np.uint32), want.view(np.uint32)), (rows, cols, t)


def test_noalloc_first_call_recorded_in_a_graph(q8rt, rt):
    """A runtime of its own whose first product is rt_gemm_dev_noalloc on a K-split shape, recorded
    into a graph: anything that would allocate while a graph is being recorded stops the process
    with the reason (the runtime's workspaces, the matrix-core partials among them, grow only
    outside a recording), so a recording that completes shows the entry allocates nothing. Three
    replays, with eager work of the same runtime between them, each bit for bit rt_gemm_dev's."""
    rows, cols, t = 12288, 4096, 40
    rng = np.random.default_rng(808)
    q8 = synth.q8_rows(rng, rows, cols)
    x = synth.x_f32(rng, t, cols)
    w = rt.upload(q8, rows, cols)
    try:
        want = _product(rt, rt.lib.rt_gemm_dev, w, rows, cols, x)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    r2 = q8rt.Runtime()
    try:
        w2 = r2.upload(q8, rows, cols)
        dx, dy = r2.alloc(x.nbytes), r2.alloc(4 * t * rows)
        r2.to_dev(dx, x)
        print("noalloc: recording its first product", flush=True)
        r2.lib.rt_graph_begin(r2.R)
        r2.lib.rt_gemm_dev_noalloc(r2.R, c.c_void_p(w2), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dy))
        g = r2.lib.rt_graph_end(r2.R)
        for i in range(3):
            r2.to_dev(dy, np.full((t, rows), np.nan, np.float32))
            r2.lib.rt_graph_launch(r2.R, c.c_void_p(g))
            y = np.empty((t, rows), np.float32)
            r2.from_dev(y, dy)
            assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), f"replay {i}"
        r2.lib.rt_graph_free(r2.R, c.c_void_p(g))
        r2.free(dx)
        r2.free(dy)
        r2.lib.rt_q8_free(r2.R, c.c_void_p(w2))
    finally:
        r2.close()
