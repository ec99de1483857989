"""The epilogues on either side of a product (src/apl/qwen35.apl:49, 131-139) on the GPU: the RMS norm
that makes a layer's x, fused into the decode products (plain, the gate+up pair, the round) or run
apart, and the residual added after W_OUT / W_DOWN.

Bars: the norm alone against the F64 oracle within F32 error (max |err| <= 1e-6 of the largest
output); a product on the normed x against the F64 product of the F64-normed x with the parity bar
of tests/parity.py (NRMSE <= 1e-5, max rel <= 1e-4); the residual bit for bit against the product
plus one F32 add, and against F64 with the parity bar. Shapes cover the fused kernels (K = 2048,
4096, 12288) and ones that run apart (K = 1024, 3072; t >= 5 on the matrix cores)."""
import ctypes as c

import numpy as np
import pytest

import synth
from parity import assert_parity
from test_gpu_parity import Dev, gpu_gemm

pytestmark = pytest.mark.gpu
EPS = 1e-6


def say(*a):
    print(*a, flush=True)


def _vec(seed, cols):
    rng = np.random.default_rng(seed)
    return (1 + 0.2 * rng.standard_normal(cols)).astype(np.float32)


@pytest.mark.parametrize("cols", [96, 1024, 4096, 12288])
def test_rmsnorm_dev(rt, oracle, reference, cols):
    """rt_rmsnorm_dev against the F64 norm, and the reference's own F32 norm where it is built."""
    t = 3
    rng = np.random.default_rng(cols)
    x = (2 * rng.standard_normal((t, cols))).astype(np.float32)
    x[1] *= 1e-3
    nw = _vec(cols + 1, cols)
    with Dev(rt) as d:
        dx, dn, do = d.put(x), d.put(nw), d.empty(4 * t * cols)
        rt.lib.rt_rmsnorm_dev(rt.R, c.c_void_p(dx), cols, t, cols, c.c_void_p(dn), EPS, c.c_void_p(do))
        got = d.get(do, (t, cols), np.float32)
        # in place (xn = x)
        rt.lib.rt_rmsnorm_dev(rt.R, c.c_void_p(dx), cols, t, cols, c.c_void_p(dn), EPS, c.c_void_p(dx))
        inplace = d.get(dx, (t, cols), np.float32)
    ref = oracle.rmsnorm_f64(x, nw, EPS)
    for i in range(t):
        assert np.max(np.abs(got[i] - ref[i])) <= 1e-6 * np.max(np.abs(ref[i])), i
        if reference is not None:
            r32 = reference.rmsnorm_f32(x[i], nw, EPS)
            assert np.max(np.abs(got[i] - r32)) <= 1e-6 * np.max(np.abs(r32)), i
    assert np.array_equal(inplace, got)


NORM_SHAPES = [(4096, 4096), (2048, 2048), (1024, 12288), (512, 3072), (256, 1024)]


@pytest.mark.parametrize("rows,cols", NORM_SHAPES)
@pytest.mark.parametrize("t", [1, 2, 4, 6])
def test_product_on_normed_x(rt, oracle, rows, cols, t):
    """rt_gemm_norm_dev: Y = RMS(X) W^T, fused (decode, K of the layers) or apart (other K, t >= 5),
    against the F64 product of the F64-normed x; and close to the norm then the product."""
    say(f"norm product {rows}x{cols} t={t}")
    q8, x = synth.case(7 * rows + cols + t, rows, cols, t)
    nw = _vec(rows + t, cols)
    w = rt.upload(q8, rows, cols)
    try:
        with Dev(rt) as d:
            dx, dn, dy = d.put(x), d.put(nw), d.empty(4 * t * rows)
            rt.lib.rt_gemm_norm_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dn), EPS, c.c_void_p(dy))
            y = d.get(dy, (t, rows), np.float32)
            dxn = d.empty(4 * t * cols)
            rt.lib.rt_rmsnorm_dev(rt.R, c.c_void_p(dx), cols, t, cols, c.c_void_p(dn), EPS, c.c_void_p(dxn))
            xn = d.get(dxn, (t, cols), np.float32)
        apart = gpu_gemm(rt, q8, rows, cols, xn, w=w)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    ref = oracle.gemm_f64d(q8, rows, cols, oracle.rmsnorm_f64(x, nw, EPS))
    assert_parity(y, ref, f"norm product {rows}x{cols} t={t}")
    assert_parity(apart, ref, f"norm then product {rows}x{cols} t={t}")


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1536, 2048), (512, 3072)])
@pytest.mark.parametrize("t", [1, 3, 4, 8])
def test_pair_on_normed_x(rt, oracle, rows, cols, t):
    """rt_gemv_swiglu_norm_dev: SiLU(RMS(X) Wg^T) * (RMS(X) Wu^T) against F64."""
    say(f"norm pair {rows}x{cols} t={t}")
    qg, x = synth.case(11 * rows + t, rows, cols, t)
    qu, _ = synth.case(13 * rows + t, rows, cols, 1)
    nw = _vec(rows, cols)
    wg, wu = rt.upload(qg, rows, cols), rt.upload(qu, rows, cols)
    try:
        with Dev(rt) as d:
            dx, dn, dy = d.put(x), d.put(nw), d.empty(4 * t * rows)
            rt.lib.rt_gemv_swiglu_norm_dev(rt.R, c.c_void_p(wg), c.c_void_p(wu), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dn), EPS,
                                           c.c_void_p(dy))
            y = d.get(dy, (t, rows), np.float32)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(wg))
        rt.lib.rt_q8_free(rt.R, c.c_void_p(wu))
    xn = oracle.rmsnorm_f64(x, nw, EPS)
    ref = oracle.swiglu_f64(oracle.gemm_f64d(qg, rows, cols, xn), oracle.gemm_f64d(qu, rows, cols, xn))
    assert_parity(y, ref, f"norm pair {rows}x{cols} t={t}")


@pytest.mark.parametrize("cols,t", [(4096, 1), (4096, 3), (2048, 4), (3072, 2), (4096, 7)])
def test_round_on_normed_x(rt, oracle, cols, t):
    """rt_gemv_round_norm_dev: the DeltaNet quartet's shapes (and a K the fused round does not take,
    and t >= 5) sharing RMS(X), against F64 product by product."""
    say(f"norm round K={cols} t={t}")
    shapes = [8192 if cols == 4096 else 1024, 4096 if cols == 4096 else 512, 32, 32]
    q8s, x = [], None
    for i, r in enumerate(shapes):
        q, xx = synth.case(100 * i + cols + t, r, cols, t)
        q8s.append(q)
        x = xx if x is None else x
    nw = _vec(cols + 3, cols)
    ws = [rt.upload(q, r, cols) for q, r in zip(q8s, shapes)]
    try:
        with Dev(rt) as d:
            dx, dn = d.put(x), d.put(nw)
            dys = [d.empty(4 * t * r) for r in shapes]
            warr = (c.c_void_p * 4)(*ws)
            rarr = (c.c_long * 4)(*shapes)
            yarr = (c.c_void_p * 4)(*dys)
            rt.lib.rt_gemv_round_norm_dev(rt.R, 4, warr, rarr, cols, c.c_void_p(dx), cols, t, c.c_void_p(dn), EPS, yarr)
            ys = [d.get(p, (t, r), np.float32) for p, r in zip(dys, shapes)]
    finally:
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    xn = oracle.rmsnorm_f64(x, nw, EPS)
    for q, r, y in zip(q8s, shapes, ys):
        assert_parity(y, oracle.gemm_f64d(q, r, cols, xn), f"norm round {r}x{cols} t={t}")


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (4096, 12288), (2048, 2048), (512, 3072), (256, 1024)])
@pytest.mark.parametrize("t", [1, 4, 5, 16, 40])
def test_residual(rt, oracle, rows, cols, t):
    """rt_gemm_residual_dev: Y = R + X W^T, fused (decode kernel, matrix-core store or partial sum)
    or apart; bit for bit the product plus one F32 add, in place too, and against F64."""
    say(f"residual {rows}x{cols} t={t}")
    q8, x = synth.case(17 * rows + cols + t, rows, cols, t)
    r = np.random.default_rng(rows + t).standard_normal((t, rows)).astype(np.float32)
    w = rt.upload(q8, rows, cols)
    try:
        with Dev(rt) as d:
            dx, dr, dy = d.put(x), d.put(r), d.empty(4 * t * rows)
            rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dr), c.c_void_p(dy))
            y = d.get(dy, (t, rows), np.float32)
            rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dr), c.c_void_p(dr))
            inplace = d.get(dr, (t, rows), np.float32)
        plain = gpu_gemm(rt, q8, rows, cols, x, w=w)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    assert np.array_equal(y.view(np.uint32), (r + plain).view(np.uint32))
    assert np.array_equal(inplace.view(np.uint32), y.view(np.uint32))
    assert_parity(y, r.astype(np.float64) + oracle.gemm_f64(q8, rows, cols, x), f"residual {rows}x{cols} t={t}")


def test_layer_graph_with_epilogues(rt, oracle):
    """A 2B-shaped FFN half-layer with its epilogues, recorded as a graph: h = SiLU(RMS(X) Wg^T) *
    (RMS(X) Wu^T), X <- X + h Wd^T, replayed three times with eager work between; every replay's
    bits equal the eager run's, and the eager run meets the parity bar against F64."""
    H, F, t = 2048, 6144, 1
    qg, x = synth.case(501, F, H, t)
    qu, _ = synth.case(502, F, H, 1)
    qd, _ = synth.case(503, H, F, 1)
    nw = _vec(504, H)
    wg, wu, wd = rt.upload(qg, F, H), rt.upload(qu, F, H), rt.upload(qd, H, F)
    try:
        with Dev(rt) as d:
            dx0, dn, dh, dx = d.put(x), d.put(nw), d.empty(4 * F * t), d.empty(4 * H * t)

            def layer():
                rt.lib.rt_gemv_swiglu_norm_dev(rt.R, c.c_void_p(wg), c.c_void_p(wu), F, H, c.c_void_p(dx), H, t, c.c_void_p(dn), EPS, c.c_void_p(dh))
                rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(wd), H, F, c.c_void_p(dh), F, t, c.c_void_p(dx), c.c_void_p(dx))

            rt.lib.rt_dev_copy(rt.R, c.c_void_p(dx), c.c_void_p(dx0), 4 * H * t)
            layer()
            eager = d.get(dx, (t, H), np.float32)
            rt.lib.rt_graph_begin(rt.R)
            layer()
            g = rt.lib.rt_graph_end(rt.R)
            try:
                for k in range(3):
                    rt.lib.rt_dev_copy(rt.R, c.c_void_p(dx), c.c_void_p(dx0), 4 * H * t)
                    rt.lib.rt_graph_launch(rt.R, c.c_void_p(g))
                    got = d.get(dx, (t, H), np.float32)
                    assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), k
                    layer()  # eager work between the replays
                    rt.sync()
            finally:
                rt.lib.rt_graph_free(rt.R, c.c_void_p(g))
    finally:
        for w in (wg, wu, wd):
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    xn = oracle.rmsnorm_f64(x, nw, EPS)
    h = oracle.swiglu_f64(oracle.gemm_f64d(qg, F, H, xn), oracle.gemm_f64d(qu, F, H, xn))
    ref = x.astype(np.float64) + oracle.gemm_f64d(qd, H, F, h)
    assert_parity(eager, ref, "FFN half-layer with epilogues")


def test_epilogues_apart_switch(rt, oracle):
    """rt_set_epi_apart(R, 1) runs the epilogues as kernels of their own: the residual's bits are the
    fused ones, the norm product meets the bar (its sum in the separate kernel's order)."""
    rows, cols, t = 4096, 4096, 2
    q8, x = synth.case(909, rows, cols, t)
    nw = _vec(910, cols)
    r = np.random.default_rng(911).standard_normal((t, rows)).astype(np.float32)
    w = rt.upload(q8, rows, cols)
    out = {}
    try:
        for apart in (False, True):
            old = rt.set_epi_apart(apart)
            try:
                with Dev(rt) as d:
                    dx, dn, dr, dy, dz = d.put(x), d.put(nw), d.put(r), d.empty(4 * t * rows), d.empty(4 * t * rows)
                    rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dr), c.c_void_p(dy))
                    rt.lib.rt_gemm_norm_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dn), EPS, c.c_void_p(dz))
                    out[apart] = (d.get(dy, (t, rows), np.float32), d.get(dz, (t, rows), np.float32))
            finally:
                rt.set_epi_apart(old)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    assert np.array_equal(out[False][0].view(np.uint32), out[True][0].view(np.uint32))
    ref = oracle.gemm_f64d(q8, rows, cols, oracle.rmsnorm_f64(x, nw, EPS))
    assert_parity(out[True][1], ref, "norm product apart")
    assert_parity(out[False][1], ref, "norm product fused")


def _random_epilogue_cases(n=16, seed=77):
    """seeded shapes: rows a multiple of 16, cols a multiple of 32 (odd block counts, K of the fused
    kernels and others), t across decode and matrix-core counts"""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        rows = 16 * int(rng.integers(1, 81))
        cols = int(rng.choice([2048, 4096, 12288])) if i % 4 == 0 else 32 * int(rng.integers(1, 97))
        t = int(rng.choice([1, 2, 3, 4, 5, 9, 16, 23]))
        out.append((i, rows, cols, t))
    return out


@pytest.mark.parametrize("case", _random_epilogue_cases(), ids=lambda c: f"{c[1]}x{c[2]}t{c[3]}")
def test_epilogues_random_shapes(rt, oracle, case):
    """The norm before and the residual after a product on seeded random shapes, whichever route the
    shape takes (fused into the decode or matrix-core kernel, or apart): the norm product at the
    parity bar against F64, the residual bit for bit against the product plus one F32 add, in place
    too."""
    i, rows, cols, t = case
    say(f"random epilogues {rows}x{cols} t={t}")
    q8, x = synth.case(5000 + i, rows, cols, t)
    nw = _vec(6000 + i, cols)
    r = np.random.default_rng(7000 + i).standard_normal((t, rows)).astype(np.float32)
    w = rt.upload(q8, rows, cols)
    try:
        with Dev(rt) as d:
            dx, dn, dr, dy = d.put(x), d.put(nw), d.put(r), d.empty(4 * t * rows)
            rt.lib.rt_gemm_norm_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dn), EPS, c.c_void_p(dy))
            yn = d.get(dy, (t, rows), np.float32)
            rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dr), c.c_void_p(dy))
            yr = d.get(dy, (t, rows), np.float32)
            rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dr), c.c_void_p(dr))
            inplace = d.get(dr, (t, rows), np.float32)
        plain = gpu_gemm(rt, q8, rows, cols, x, w=w)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    assert_parity(yn, oracle.gemm_f64d(q8, rows, cols, oracle.rmsnorm_f64(x, nw, EPS)), f"norm product {rows}x{cols} t={t}")
    assert np.array_equal(yr.view(np.uint32), (r + plain).view(np.uint32))
    assert np.array_equal(inplace.view(np.uint32), yr.view(np.uint32))
