"""GPU parity: the HIP kernels through the C-ABI against the oracle. Every test here needs the MI355X.

  - the primitive conversions reproduce the reference's gate 2.1 lanes;
  - the GPU repack writes form S byte for byte;
  - the reference-order kernels are bit-identical to the reference's own products (fixtures made
    from its compiled sources) and to the oracle at the configurations' shapes;
  - the fast kernels meet NRMSE <= 1e-5 and max rel <= 1e-4 (tests/parity.py) against the F64
    closed form, at every configuration's shape and token count, and are deterministic;
  - the host-pointer entry points (rt_gemv, rt_gemm, the queued round) equal the device ones.
"""
import ctypes as c
import os
import subprocess
import sys

import numpy as np
import pytest

import synth
from parity import assert_parity, metrics

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def say(*a):
    print(*a, flush=True)


class Dev:
    """Device buffers for one product, freed on exit."""

    def __init__(self, rt):
        self.rt, self.bufs = rt, []

    def put(self, a):
        p = self.rt.alloc(max(a.nbytes, 16))
        self.rt.to_dev(p, a)
        self.bufs.append(p)
        return p

    def empty(self, nbytes):
        p = self.rt.alloc(max(nbytes, 16))
        self.bufs.append(p)
        return p

    def get(self, p, shape, dtype):
        a = np.empty(shape, dtype)
        self.rt.from_dev(a, p)
        return a

    def __enter__(self):
        return self

    def __exit__(self, *e):
        for p in self.bufs:
            self.rt.free(p)


def gpu_gemm(rt, q8, rows, cols, x, exact=False, w=None):
    """Y [t rows] = X W^T through rt_q8_upload + rt_gemm_dev."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    t = x.shape[0]
    old = rt.set_exact(exact)
    try:
        own = w is None
        if own:
            w = rt.upload(q8, rows, cols)
        with Dev(rt) as d:
            dx, dy = d.put(x), d.empty(4 * t * rows)
            rt.lib.rt_gemm_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dy))
            y = d.get(dy, (t, rows), np.float32)
        if own:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    finally:
        rt.set_exact(old)
    return y


def gpu_swiglu(rt, q8g, q8u, rows, cols, x, exact=False):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    t = x.shape[0]
    old = rt.set_exact(exact)
    wg, wu = rt.upload(q8g, rows, cols), rt.upload(q8u, rows, cols)
    try:
        with Dev(rt) as d:
            dx, dy = d.put(x), d.empty(4 * t * rows)
            rt.lib.rt_gemv_swiglu_dev(rt.R, c.c_void_p(wg), c.c_void_p(wu), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(dy))
            y = d.get(dy, (t, rows), np.float32)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(wg))
        rt.lib.rt_q8_free(rt.R, c.c_void_p(wu))
        rt.set_exact(old)
    return y


def test_device_is_gfx950(rt):
    name, cus = rt.device_info()
    say("device:", name, "CUs:", cus)
    assert "gfx950" in name


def test_primitive_gate21_lanes(rt, oracle):
    """The int8 and binary16 converts and the fma of the product kernels, on the reference's gate 2.1
    inputs: the s8 lanes hash to the golden line (gate-2.1.txt:1); the f16 lanes (all 65536 patterns,
    twice) equal the oracle's bit for bit except NaN payload quieting, and hash to the golden line
    when no NaN lane differs."""
    q, h, x8, c8, xf, cf = oracle.gate21_inputs()
    s8_want, f16_want = oracle.gate21_arrays()
    with Dev(rt) as d:
        pq, ph, px8, pc8, pxf, pcf = (d.put(a) for a in (q, h, x8, c8, xf, cf))
        po8, pof = d.empty(4 * 512), d.empty(4 * 131072)
        rt.lib.rt_prims_dev(rt.R, c.c_void_p(pq), c.c_void_p(px8), c.c_void_p(pc8), c.c_void_p(po8), 512, c.c_void_p(ph), c.c_void_p(pxf),
                            c.c_void_p(pcf), c.c_void_p(pof), 131072)
        s8 = d.get(po8, 512, np.float32)
        f16 = d.get(pof, 131072, np.float32)
    golden = {l.split()[0]: l.split()[4] for l in open(os.path.join(GOLDEN, "gate-2.1.txt")) if l.strip()}
    assert f"{oracle.hash(s8):016x}" == golden["s8"]
    assert np.array_equal(s8.view(np.uint32), s8_want.view(np.uint32))
    nan = np.isnan(f16_want)
    assert np.array_equal(np.isnan(f16), nan)
    assert np.array_equal(f16[~nan].view(np.uint32), f16_want[~nan].view(np.uint32))
    quiet_only = np.all((f16[nan].view(np.uint32) ^ f16_want[nan].view(np.uint32)) & ~np.uint32(0x00400000) == 0)
    say("f16 gate: NaN lanes", int(nan.sum()), "payload kept up to the quiet bit:", bool(quiet_only),
        "hash", f"{oracle.hash(f16):016x}", "golden", golden["f16"])
    if np.array_equal(f16.view(np.uint32), f16_want.view(np.uint32)):
        assert f"{oracle.hash(f16):016x}" == golden["f16"]


@pytest.mark.parametrize("rows,cols", [(16, 32), (48, 96), (64, 512), (4096, 4096)])
def test_repack_on_device(rt, oracle, rows, cols):
    q8, _ = synth.case(rows * 7 + cols, rows, cols, 1)
    with Dev(rt) as d:
        src, dst = d.put(q8), d.empty(q8.nbytes)
        rt.lib.rt_q8_repack_dev(rt.R, c.c_void_p(src), rows, cols, c.c_void_p(dst))
        got = d.get(dst, q8.size, np.uint8)
    assert np.array_equal(got, oracle.repack_s(q8, rows, cols))


def fixtures():
    z = np.load(os.path.join(GOLDEN, "ref_products.npz"))
    for i in range(int(z["ncases"][0])):
        seed, rows, cols, t, logn = (int(v) for v in z[f"c{i}_meta"])
        yield (seed, rows, cols, t), z[f"c{i}_q8"], z[f"c{i}_x"], z[f"c{i}_y"]


def test_exact_kernels_equal_reference_fixtures(rt):
    """The reference-order kernels reproduce the reference's own gemv/gemm outputs bit for bit, and
    config 1 (4096x4096, seed 0)."""
    for case, q8, x, y in fixtures():
        say("fixture", case)
        got = gpu_gemm(rt, q8, case[1], case[2], x, exact=True)
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), case
    z = np.load(os.path.join(GOLDEN, "ref_products.npz"))
    q8, x = synth.case(0, 4096, 4096, 1)
    got = gpu_gemm(rt, q8, 4096, 4096, x, exact=True)[0]
    assert np.array_equal(got.view(np.uint32), z["cfg1_y"].view(np.uint32))


def test_fast_kernels_on_fixtures(rt, oracle):
    for case, q8, x, y in fixtures():
        got = gpu_gemm(rt, q8, case[1], case[2], x)
        m = assert_parity(got, oracle.gemm_f64(q8, case[1], case[2], x), f"fixture {case}")
        assert_parity(got, y.astype(np.float64), f"fixture {case} vs the reference's F32")
        say("fast", case, m)


# the configurations' matrices: 2B layer (QKV, out, gate/up, down), 9B layer, and config 1; then the
# 9B model's other per-layer matrices (src/apl/qwen35.apl:93-97, 117-120): DeltaNet QKV and attention
# Q (8192 rows), attention K and V (1024), the DeltaNet beta and alpha (32)
SHAPES = [(3072, 2048), (2048, 2048), (6144, 2048), (2048, 6144), (6144, 4096), (4096, 4096), (12288, 4096), (4096, 12288),
          (8192, 4096), (1024, 4096), (32, 4096)]


@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("t", [1, 2, 3, 4])
def test_fast_gemv_shapes(rt, oracle, rows, cols, t):
    dist = "lognormal" if t > 1 else "normal"
    q8, x = synth.case(rows + cols + t, rows, cols, t, dist)
    say("gemv", rows, cols, t, dist)
    got = gpu_gemm(rt, q8, rows, cols, x)
    m = assert_parity(got, oracle.gemm_f64(q8, rows, cols, x), f"{rows}x{cols} t={t}")
    say("  ", m)


@pytest.mark.parametrize("t", [5, 8, 16, 17, 40, 64])
def test_fast_gemm_tokens(rt, oracle, t):
    rows, cols = 1024, 4096
    q8, x = synth.case(300 + t, rows, cols, t)
    say("gemm", rows, cols, t)
    got = gpu_gemm(rt, q8, rows, cols, x)
    assert_parity(got, oracle.gemm_f64(q8, rows, cols, x), f"gemm t={t}")


@pytest.mark.parametrize("rows,cols", [(12288, 4096), (4096, 12288)])
def test_fast_gemm_prompt_shapes(rt, oracle, rows, cols):
    """The prompt configuration: M = 16 and 40 on the 9B FFN matrices."""
    for t in (16, 40):
        q8, x = synth.case(rows + t, rows, cols, t)
        say("prompt gemm", rows, cols, t)
        got = gpu_gemm(rt, q8, rows, cols, x)
        assert_parity(got, oracle.gemm_f64(q8, rows, cols, x), f"{rows}x{cols} t={t}")


@pytest.mark.parametrize("rows,cols", [(12288, 4096), (6144, 2048)])
@pytest.mark.parametrize("t", [1, 2, 3, 4])
def test_fused_gate_up(rt, oracle, rows, cols, t):
    """SiLU(G) * U for the 9B and 2B FFN pairs (2 x 12288x4096, 2 x 6144x2048: 8, 4 and 2 rows a
    workgroup), heavy-tailed scales."""
    rng = np.random.default_rng(900 + t + rows)
    q8g = synth.q8_rows(rng, rows, cols, "lognormal")
    q8u = synth.q8_rows(rng, rows, cols, "lognormal")
    x = synth.x_f32(rng, t, cols)
    say("swiglu", rows, cols, t)
    got = gpu_swiglu(rt, q8g, q8u, rows, cols, x)
    want = oracle.swiglu_f64(oracle.gemm_f64(q8g, rows, cols, x), oracle.gemm_f64(q8u, rows, cols, x))
    m = assert_parity(got, want, f"swiglu t={t}")
    say("  ", m)
    ex = gpu_swiglu(rt, q8g, q8u, rows, cols, x, exact=True)
    assert_parity(ex, want, f"exact swiglu t={t}")


@pytest.mark.parametrize("rows,cols,t", [(1888, 512, 16), (48, 4096, 33), (16, 1024, 5), (4096, 12288, 64), (1024, 2048, 100), (6144, 4096, 24),
                                         (256, 256, 47)])
def test_matrix_core_gemm_shapes(rt, oracle, rows, cols, t):
    """The matrix-core product at row counts that leave a partial workgroup (1888, 48, 16), every token
    tile count (5..64), more than 64 tokens (two launches), and heavy-tailed scales on one case; the K
    split's partials are summed in split order by a second kernel."""
    dist = "lognormal" if t == 24 else "normal"
    q8, x = synth.case(rows * 3 + cols + t, rows, cols, t, dist)
    say("mfma gemm", rows, cols, t, dist)
    got = gpu_gemm(rt, q8, rows, cols, x)
    m = assert_parity(got, oracle.gemm_f64(q8, rows, cols, x), f"{rows}x{cols} t={t}")
    say("  ", m)


def test_matrix_core_gemm_deterministic(rt):
    """The K-split sums partials in split order: repeated products give the same bits."""
    rows, cols, t = 4096, 12288, 16
    q8, x = synth.case(17, rows, cols, t)
    w = rt.upload(q8, rows, cols)
    ys = [gpu_gemm(rt, q8, rows, cols, x, w=w) for _ in range(3)]
    rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    for y in ys[1:]:
        assert np.array_equal(y.view(np.uint32), ys[0].view(np.uint32))


class force:
    """The matrix-core product's K split (ks > 0) and, with streaming, its streaming kernel for one
    token tile, for a block (rt_gemm_force; the planner's choices again after it)."""

    def __init__(self, rt, streaming=False, ks=0):
        self.rt, self.streaming, self.ks = rt, streaming, ks

    def __enter__(self):
        self.rt.gemm_force(self.streaming, self.ks)

    def __exit__(self, *e):
        self.rt.gemm_force()


@pytest.mark.parametrize("rows,cols,t", [(12288, 4096, 16), (4096, 12288, 9), (1888, 1056, 5), (48, 4096, 13)])
def test_x_resident_gemm_equals_streaming(rt, oracle, rows, cols, t):
    """One token tile: the x-resident kernel (the default at t <= 16) and the streaming kernel with
    the same ranges (gemm_mfma<1, 1, 2, 16>) give the same bits on the same K split. One K split
    gives the x-resident kernel several LDS segments (every range of K in one workgroup: 4, 12 and
    2 segments here) and stores Y directly; 1056 columns end on half a pair; 1888 and 48 rows leave
    waves past the last row tile."""
    q8, x = synth.case(5 * rows + cols + t, rows, cols, t)
    w = rt.upload(q8, rows, cols)
    try:
        for ks in (0, 1, 3):
            with force(rt, ks=ks):
                say("x-resident gemm", rows, cols, t, "ks", ks or "planned")
                a = gpu_gemm(rt, q8, rows, cols, x, w=w)
            with force(rt, streaming=True, ks=ks):
                b = gpu_gemm(rt, q8, rows, cols, x, w=w)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"ks {ks or 'planned'}"
            assert_parity(a, oracle.gemm_f64(q8, rows, cols, x), f"{rows}x{cols} t={t} ks {ks or 'planned'}")
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


@pytest.mark.parametrize("ks", [0, 1])
def test_x_resident_gemm_strided_x_and_residual(rt, ks):
    """x rows wider than the product (x_stride > cols) give the contiguous x's bits, and the residual
    epilogue, fused into the x-resident kernel's store (one K split) or into the partial sum, is
    the product plus one F32 add."""
    rows, cols, t, xs = 1024, 2048, 7, 2048 + 96
    q8, x = synth.case(4242, rows, cols, t)
    wide = np.full((t, xs), np.nan, np.float32)
    wide[:, :cols] = x
    r = np.random.default_rng(5).standard_normal((t, rows)).astype(np.float32)
    w = rt.upload(q8, rows, cols)
    try:
        with force(rt, ks=ks), Dev(rt) as d:
            plain = gpu_gemm(rt, q8, rows, cols, x, w=w)
            dx, dr, dy = d.put(wide), d.put(r), d.empty(4 * t * rows)
            rt.lib.rt_gemm_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), xs, t, c.c_void_p(dy))
            strided = d.get(dy, (t, rows), np.float32)
            rt.lib.rt_gemm_residual_dev(rt.R, c.c_void_p(w), rows, cols, c.c_void_p(dx), xs, t, c.c_void_p(dr), c.c_void_p(dy))
            resid = d.get(dy, (t, rows), np.float32)
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    assert np.array_equal(strided.view(np.uint32), plain.view(np.uint32))
    assert np.array_equal(resid.view(np.uint32), (r + plain).view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(12288, 4096), (2048, 2048), (16, 128)])
def test_fused_pair_many_tokens(rt, oracle, rows, cols):
    """rt_gemv_swiglu_dev at t >= 5: 64 tokens at a time, the gate and up products as one round,
    with their sums and SiLU(g)*u in one launch. A token's bits do not depend on t, so the first
    tokens at t = 70 (a 64-token round and a 6-token one) equal t = 5, 16, 64, 65 and 68 bit for bit
    (the last two end with a round of 1 and 4 tokens), and every result meets the parity bar against
    F64 (the first 8 tokens on 12288 x 4096). 16 x 128 has one K split: its products write their
    sums themselves."""
    rng = np.random.default_rng(77 + rows)
    q8g, q8u = synth.q8_rows(rng, rows, cols), synth.q8_rows(rng, rows, cols)
    x = synth.x_f32(rng, 70, cols)
    y70 = gpu_swiglu(rt, q8g, q8u, rows, cols, x)
    for t in (5, 16, 64, 65, 68):
        yt = gpu_swiglu(rt, q8g, q8u, rows, cols, x[:t])
        assert np.array_equal(yt.view(np.uint32), y70[:t].view(np.uint32)), t
    tc = 8 if rows * cols > 1 << 24 else 70
    want = oracle.swiglu_f64(oracle.gemm_f64(q8g, rows, cols, x[:tc]), oracle.gemm_f64(q8u, rows, cols, x[:tc]))
    assert_parity(y70[:tc], want, f"swiglu {rows}x{cols}")


def test_graph_replays_match_eager(rt):
    """A recorded sequence (decode products, the fused pair, and K-split matrix-core products at 16
    tokens (x-resident, 32 splits) and 40 (streaming), whose partials every run writes before it
    sums them) replayed three times, with eager work between the replays, gives the eager result
    bit for bit every time."""
    rng = np.random.default_rng(8)
    rows, cols, t, t2 = 2048, 4096, 16, 40
    mats = [synth.q8_rows(rng, rows, cols) for _ in range(3)]
    x = synth.x_f32(rng, t2, cols)
    ws = [rt.upload(m, rows, cols) for m in mats]
    with Dev(rt) as d:
        dx = d.put(x)
        y1, y2, y3, y4 = d.empty(4 * rows), d.empty(4 * 2 * rows), d.empty(4 * t * rows), d.empty(4 * t2 * rows)
        yz = d.empty(4 * t * rows)
        outs = ((y1, rows), (y2, 2 * rows), (y3, t * rows), (y4, t2 * rows))

        def seq():
            rt.lib.rt_gemm_dev(rt.R, c.c_void_p(ws[0]), rows, cols, c.c_void_p(dx), cols, 1, c.c_void_p(y1))
            rt.lib.rt_gemv_swiglu_dev(rt.R, c.c_void_p(ws[1]), c.c_void_p(ws[2]), rows, cols, c.c_void_p(dx), cols, 2, c.c_void_p(y2))
            rt.lib.rt_gemm_dev(rt.R, c.c_void_p(ws[2]), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(y3))
            rt.lib.rt_gemm_dev(rt.R, c.c_void_p(ws[1]), rows, cols, c.c_void_p(dx), cols, t2, c.c_void_p(y4))

        seq()
        want = [d.get(p, n, np.float32) for p, n in outs]
        rt.lib.rt_graph_begin(rt.R)
        seq()
        g = rt.lib.rt_graph_end(rt.R)
        try:
            for rep in range(3):
                for p, n in outs:
                    rt.to_dev(p, np.zeros(n, np.float32))
                rt.lib.rt_graph_launch(rt.R, c.c_void_p(g))
                got = [d.get(p, n, np.float32) for p, n in outs]
                for a, b in zip(got, want):
                    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"replay {rep}"
                # eager work between replays: another K-split product on the same workspace
                rt.lib.rt_gemm_dev(rt.R, c.c_void_p(ws[0]), rows, cols, c.c_void_p(dx), cols, t, c.c_void_p(yz))
                rt.sync()
        finally:
            rt.lib.rt_graph_free(rt.R, c.c_void_p(g))
            for w in ws:
                rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


@pytest.mark.parametrize("shapes", [[8192, 4096, 32, 32], [8192, 1024, 1024]], ids=["deltanet_quartet", "attention_qkv"])
@pytest.mark.parametrize("t", [1, 3])
def test_round_one_launch_equals_singles(rt, oracle, t, shapes):
    """The 9B DeltaNet quartet (QKV 8192x4096, GATE 4096x4096, BETA and ALPHA 32x4096, all reading H;
    src/apl/qwen35.apl:93-96) and the attention layer's Q, K and V (8192, 1024 and 1024 x 4096;
    qwen35.apl:117-119) as one launch (rt_gemv_round_dev) give each product's bits as its own
    launch does, and meet the parity bar."""
    cols = 4096
    n = len(shapes)
    rng = np.random.default_rng(60 + t + n)
    mats = [synth.q8_rows(rng, r, cols) for r in shapes]
    x = synth.x_f32(rng, t, cols)
    ws = [rt.upload(m, r, cols) for m, r in zip(mats, shapes)]
    try:
        singles = [gpu_gemm(rt, m, r, cols, x, w=w) for m, r, w in zip(mats, shapes, ws)]
        with Dev(rt) as d:
            dx = d.put(x)
            ys = [d.empty(4 * t * r) for r in shapes]
            W = (c.c_void_p * n)(*ws)
            R = (c.c_long * n)(*shapes)
            Y = (c.c_void_p * n)(*ys)
            rt.lib.rt_gemv_round_dev(rt.R, n, W, R, cols, c.c_void_p(dx), cols, t, Y)
            got = [d.get(p, (t, r), np.float32) for p, r in zip(ys, shapes)]
        for g, s1, m, r in zip(got, singles, mats, shapes):
            assert np.array_equal(g.view(np.uint32), s1.view(np.uint32)), r
            assert_parity(g, oracle.gemm_f64(m, r, cols, x), f"round {r}x{cols} t={t}")
    finally:
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


@pytest.mark.parametrize("shapes", [[8192, 4096, 32, 32], [8192, 1024, 1024], [12288, 12288]], ids=["deltanet_quartet", "attention_qkv", "ffn_pair"])
@pytest.mark.parametrize("t", [5, 16, 17, 40, 64, 65, 68, 70])
def test_matrix_core_round_equals_singles(rt, oracle, t, shapes):
    """From 5 tokens, 64 at a time, a round of products sharing x (rt_gemv_round_dev) runs as one
    matrix-core launch for the products (the x-resident kernel up to 16 tokens, the streaming one
    above, at the largest product's wave count) and one launch of the partial sums, each product on
    its own K split:
    every product's bits are those of its own rt_gemm_dev, at the parity bar, and the round's first
    kernel is a round kernel (the runtime's kernel records). The 9B DeltaNet quartet
    (qwen35.apl:93-96; its 32-row products are one row tile with 14 idle waves), the attention layer's
    Q, K, V (qwen35.apl:117-119) and a gate and up pair (12288 x 4096); at 64 tokens the quartet's
    partials outgrow the single product's workspace, so the round's own grows. At 65 and 68 tokens
    the last chunk holds 1 and 4 tokens: it runs as a matrix-core round too, as the single
    product's last chunk runs on the matrix cores."""
    cols = 4096
    n = len(shapes)
    rng = np.random.default_rng(700 + t + n)
    mats = [synth.q8_rows(rng, r, cols) for r in shapes]
    x = synth.x_f32(rng, t, cols)
    ws = [rt.upload(m, r, cols) for m, r in zip(mats, shapes)]
    try:
        singles = [gpu_gemm(rt, m, r, cols, x, w=w) for m, r, w in zip(mats, shapes, ws)]
        with Dev(rt) as d:
            dx = d.put(x)
            ys = [d.empty(4 * t * r) for r in shapes]
            W = (c.c_void_p * n)(*ws)
            R = (c.c_long * n)(*shapes)
            Y = (c.c_void_p * n)(*ys)
            (kname, _), = _kernels_launched(rt, lambda: rt.lib.rt_gemv_round_dev(rt.R, n, W, R, cols, c.c_void_p(dx), cols, t, Y))
            got = [d.get(p, (t, r), np.float32) for p, r in zip(ys, shapes)]
        say("round", shapes, t, kname)
        pair = n == 2 and shapes[0] == shapes[1]
        # the streaming pair runs on 3 and 4 token tiles (33..64 tokens, the first chunk of 65..70) of
        # 12 waves, which 12288 rows plan
        assert kname.startswith(("gemm_xres_pair<" if pair else "gemm_xres_round<") if t <= 16 else
                                ("gemm_mfma_pair<" if pair and t >= 33 else "gemm_mfma_round<"))
        for g, s1, m, r in zip(got, singles, mats, shapes):
            assert np.array_equal(g.view(np.uint32), s1.view(np.uint32)), r
            assert_parity(g, oracle.gemm_f64(m, r, cols, x), f"round {r}x{cols} t={t}")
    finally:
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


@pytest.mark.parametrize("ks", [0, 1, 3])
@pytest.mark.parametrize("rows,cols", [(12288, 4096), (4096, 4096), (48, 1056)])
def test_pair_round_equals_singles(rt, oracle, rows, cols, ks):
    """Two products of one shape (the FFN's gate and up, qwen35.apl:125) run as one pair kernel. At
    5 to 16 tokens a workgroup stages x once and streams product 0's ranges, then product 1's, with
    product 1's first loads issued during product 0's last ranges; at 40 and 64 tokens on the 12-wave
    kernels each range's x is staged once and each block's x limbs read once for both products'
    MFMAs (at 64 in ranges of one block pair: the split as twice as many ranges; 16 waves run the
    round kernel). Each product's
    bits are those of its own rt_gemm_dev, at the planner's K split and at forced splits of 1 and
    3, which give several segments a split, segments of an odd number of ranges and of one range
    (the prefetch crosses into product 1 at once); 12288 x 4096 takes the 12-wave kernels, 4096 x
    4096 the 16-wave ones, 48 x 1056 has idle waves and half a final pair of blocks."""
    rng = np.random.default_rng(900 + rows + ks)
    mats = [synth.q8_rows(rng, rows, cols) for _ in range(2)]
    ws = [rt.upload(m, rows, cols) for m in mats]
    try:
        with force(rt, ks=ks):
            for t in (5, 16, 40, 64):
                x = synth.x_f32(rng, t, cols)
                singles = [gpu_gemm(rt, m, rows, cols, x, w=w) for m, w in zip(mats, ws)]
                with Dev(rt) as d:
                    dx = d.put(x)
                    ys = [d.empty(4 * t * rows) for _ in range(2)]
                    W, R, Y = (c.c_void_p * 2)(*ws), (c.c_long * 2)(rows, rows), (c.c_void_p * 2)(*ys)
                    (kname, _), = _kernels_launched(rt, lambda: rt.lib.rt_gemv_round_dev(rt.R, 2, W, R, cols, c.c_void_p(dx), cols, t, Y))
                    got = [d.get(p, (t, rows), np.float32) for p in ys]
                say("pair round", rows, cols, "t", t, "ks", ks or "planned", kname)
                if t <= 16:
                    assert kname.startswith("gemm_xres_pair<"), kname
                else:  # the streaming pair where the plan takes 12 waves (12288 rows; others at a forced split)
                    assert kname.startswith(("gemm_mfma_pair<3, 1, 2, 12>" if t == 40 else "gemm_mfma_pair<4, 1, 1, 12>", "gemm_mfma_round<")), kname
                    assert kname.startswith("gemm_mfma_pair<") or rows != 12288 or ks, kname
                for g, s1 in zip(got, singles):
                    assert np.array_equal(g.view(np.uint32), s1.view(np.uint32)), (t, ks)
            for g, m in zip(got, mats):
                assert_parity(g, oracle.gemm_f64(m, rows, cols, x), f"pair {rows}x{cols} t=64 ks {ks or 'planned'}")
    finally:
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


def test_row_read_and_gather(rt, oracle):
    """rt_q8_row (the embedding read, the reference's signature) and rt_q8_rows_dev (a batch of rows)
    give the oracle's d * q bit for bit, including subnormal and zero scales."""
    rows, cols = 256, 2048
    q8, _ = synth.case(71, rows, cols, 1, "lognormal")
    q, d = synth.split(q8, rows, cols)
    d[3, :4] = 0
    d[5, 4:9] = np.uint16(3).view(np.float16)
    q8 = synth.join(q, d)
    w = rt.upload(q8, rows, cols)
    try:
        for r in (0, 3, 5, 17, 255):
            z = np.empty(cols, np.float32)
            rt.lib.rt_q8_row(c.c_void_p(w), cols, r, z.ctypes.data_as(c.c_void_p))
            assert np.array_equal(z.view(np.uint32), oracle.row(q8, cols, r).view(np.uint32)), r
        idx = np.array([7, 0, 255, 7, 128], np.int64)
        with Dev(rt) as dv:
            pi, pz = dv.put(idx), dv.empty(4 * cols * idx.size)
            rt.lib.rt_q8_rows_dev(rt.R, c.c_void_p(w), cols, c.c_void_p(pi), idx.size, c.c_void_p(pz))
            z = dv.get(pz, (idx.size, cols), np.float32)
        for k, r in enumerate(idx):
            assert np.array_equal(z[k].view(np.uint32), oracle.row(q8, cols, int(r)).view(np.uint32))
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


def test_next_token_on_device(rt, oracle):
    """rt_argmax_dev equals the oracle's rt_maxv + rt_index_of restatement: the 9B vocabulary
    (151936 logits), ragged sizes around the 4096-element chunks, ties and NaN entries."""
    rng = np.random.default_rng(19)
    cases = []
    for n in (1, 17, 4095, 4096, 4097, 12289, 151936):
        a = (rng.standard_normal(n) * 4).astype(np.float32)
        cases.append(a)
        t = a.copy()
        t[rng.integers(0, n, 3)] = t.max() + 1
        cases.append(t)
        if n > 2:
            u = a.copy()
            u[rng.integers(0, n, max(1, n // 7))] = np.nan
            cases.append(u)
    with Dev(rt) as dv:
        out = dv.empty(8)
        for a in cases:
            pa = dv.put(a)
            rt.lib.rt_argmax_dev(rt.R, c.c_void_p(pa), a.size, c.c_void_p(out))
            got = int(dv.get(out, 1, np.int64)[0])
            assert got == oracle.next(a), (a.size, got, oracle.next(a))


def test_exact_kernels_at_config_shapes(rt, oracle):
    """Bit-identical to the oracle (the reference's order) at the 9B shapes, tokens 1 and 3."""
    for rows, cols, t in [(4096, 12288, 1), (6144, 4096, 3)]:
        q8, x = synth.case(rows + 2 * cols + t, rows, cols, t)
        got = gpu_gemm(rt, q8, rows, cols, x, exact=True)
        assert np.array_equal(got.view(np.uint32), oracle.gemm(q8, rows, cols, x, threads=8).view(np.uint32))


def test_deterministic_and_prefix(rt):
    """Repeated products give the same bits; the first 1024 rows of a 4096-row handle (the draft
    head's use, src/apl/qwen35.apl:170-172) give the first 1024 outputs."""
    rows, cols = 4096, 4096
    q8, x = synth.case(4242, rows, cols, 2)
    w = rt.upload(q8, rows, cols)
    a = gpu_gemm(rt, q8, rows, cols, x, w=w)
    b = gpu_gemm(rt, q8, rows, cols, x, w=w)
    p = gpu_gemm(rt, q8, 1024, cols, x, w=w)
    rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(p.view(np.uint32), a[:, :1024].view(np.uint32))


HOST_MODES = {"x_copied": False, "x_direct": True}


def host_mode(rt, mode):
    """Sets how the host-pointer calls stage x (rt_set_x_direct); returns the previous setting."""
    return rt.set_x_direct(HOST_MODES[mode])


def restore_host_mode(rt, old):
    rt.set_x_direct(old)


@pytest.mark.parametrize("mode", list(HOST_MODES))
def test_host_pointer_entry_points(rt, mode):
    """rt_gemv, rt_gemm, a queued round of 4 products sharing x (open/go), a mixed round and queued
    prompt rounds (6 and 40 tokens) give the same bits as the device entry points, with x copied to
    HBM first or read by the decode kernels from the pinned staging."""
    rows, cols = 2048, 2048
    rng = np.random.default_rng(31)
    mats = [synth.q8_rows(rng, rows, cols) for _ in range(4)]
    x = synth.x_f32(rng, 6, cols)
    ws = [rt.upload(m, rows, cols) for m in mats]
    old_mode = host_mode(rt, mode)
    try:
        want1 = [gpu_gemm(rt, m, rows, cols, x[0], w=w)[0] for m, w in zip(mats, ws)]
        y = np.empty(rows, np.float32)
        rt.gemv(ws[0], rows, cols, x[0], y)
        assert np.array_equal(y.view(np.uint32), want1[0].view(np.uint32))
        ys = [np.empty(rows, np.float32) for _ in range(4)]
        rt.gemv_open()
        for w, yy in zip(ws, ys):
            rt.gemv_q(w, rows, cols, x[0], yy)
        rt.gemv_go()
        for yy, wv in zip(ys, want1):
            assert np.array_equal(yy.view(np.uint32), wv.view(np.uint32))
        for t in (2, 6):
            Y = np.empty((t, rows), np.float32)
            rt.gemm(ws[1], rows, cols, x[:t], t, Y)
            assert np.array_equal(Y.view(np.uint32), gpu_gemm(rt, mats[1], rows, cols, x[:t], w=ws[1]).view(np.uint32))
        # a mixed round: two gemv sharing x and a gemm
        Y = np.empty((6, rows), np.float32)
        rt.gemv_q(ws[2], rows, cols, x[0], ys[0])
        rt.gemm_q(ws[3], rows, cols, x, 6, Y)
        rt.gemv_q(ws[0], rows, cols, x[0], ys[1])
        rt.gemv_go()
        assert np.array_equal(ys[0].view(np.uint32), want1[2].view(np.uint32))
        assert np.array_equal(ys[1].view(np.uint32), want1[0].view(np.uint32))
        assert np.array_equal(Y.view(np.uint32), gpu_gemm(rt, mats[3], rows, cols, x, w=ws[3]).view(np.uint32))
        # prompt rounds: three queued products sharing x at 6 tokens (the x-resident round), at 40
        # (the streaming one) and at 66 (a 64-token round, then one of 2 tokens), each the bits of
        # its own device product
        for t in (6, 40, 66):
            xt = synth.x_f32(rng, t, cols)
            Ys = [np.empty((t, rows), np.float32) for _ in range(3)]
            for w, Yy in zip(ws[:3], Ys):
                rt.gemm_q(w, rows, cols, xt, t, Yy)
            rt.gemv_go()
            for Yy, m, w in zip(Ys, mats, ws):
                assert np.array_equal(Yy.view(np.uint32), gpu_gemm(rt, m, rows, cols, xt, w=w).view(np.uint32)), t
    finally:
        restore_host_mode(rt, old_mode)
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


@pytest.mark.parametrize("mode", list(HOST_MODES))
def test_host_call_waits_for_stream_work(rt, mode):
    """A host-pointer call made while the runtime's stream still repacks the matrix it reads (no
    wait between the two) sees the repacked matrix and not the fill before it."""
    rows, cols = 8192, 4096
    rng = np.random.default_rng(37)
    q8 = synth.q8_rows(rng, rows, cols)
    x = synth.x_f32(rng, 2, cols)
    src, out = rt.alloc(q8.nbytes), rt.alloc(q8.nbytes)
    old_mode = host_mode(rt, mode)
    try:
        rt.to_dev(src, q8)
        rt.lib.rt_f32_fill_dev(rt.R, c.c_void_p(out), q8.nbytes // 4, 99)
        rt.sync()
        for rep in range(3):
            rt.lib.rt_q8_repack_dev(rt.R, c.c_void_p(src), rows, cols, c.c_void_p(out))
            y = np.full(rows, np.nan, np.float32)
            rt.gemv(out, rows, cols, x[rep % 2], y)
            say("host call after queued repack", mode, rep)
            want = gpu_gemm(rt, q8, rows, cols, x[rep % 2:rep % 2 + 1])[0]
            assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
            rt.lib.rt_f32_fill_dev(rt.R, c.c_void_p(out), q8.nbytes // 4, 100 + rep)
    finally:
        restore_host_mode(rt, old_mode)
        rt.free(out)  # and with it the handle rt_q8_repack_dev registered there
        rt.free(src)


@pytest.mark.parametrize("mode", list(HOST_MODES))
def test_host_calls_alternating_x_see_each_new_x(rt, mode):
    """300 host-pointer calls back to back, x cycling through three vectors (and a round of two
    products every fourth call): each y equals, bit for bit, the device product of the x that call
    passed, so no call reads the previous call's x from a cache (the decode kernels read x from
    the pinned staging that the host rewrites before each call)."""
    rows, cols = 2048, 4096
    rng = np.random.default_rng(43)
    mats = [synth.q8_rows(rng, rows, cols) for _ in range(2)]
    xs = synth.x_f32(rng, 3, cols)
    ws = [rt.upload(m, rows, cols) for m in mats]
    old_mode = host_mode(rt, mode)
    try:
        want = [[gpu_gemm(rt, m, rows, cols, xs[k], w=w)[0] for k in range(3)] for m, w in zip(mats, ws)]
        y0, y1 = np.empty(rows, np.float32), np.empty(rows, np.float32)
        bad = []
        for i in range(300):
            k = i % 3
            if i % 4 == 3:
                rt.gemv_q(ws[0], rows, cols, xs[k], y0)
                rt.gemv_q(ws[1], rows, cols, xs[k], y1)
                rt.gemv_go()
                ok = np.array_equal(y0.view(np.uint32), want[0][k].view(np.uint32)) and np.array_equal(y1.view(np.uint32), want[1][k].view(np.uint32))
            else:
                rt.gemv(ws[i % 2], rows, cols, xs[k], y0)
                ok = np.array_equal(y0.view(np.uint32), want[i % 2][k].view(np.uint32))
            if not ok:
                bad.append(i)
        say("alternating x", mode, "calls 300, mismatches", len(bad))
        assert not bad, bad[:10]
    finally:
        restore_host_mode(rt, old_mode)
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


@pytest.mark.parametrize("mode", list(HOST_MODES))
def test_host_pointer_staging_grows_and_refreshes(rt, mode):
    """The host-pointer products store y into pinned staging that grows with the call: a sequence of
    growing shapes and token counts (up to 70 tokens, two matrix-core launches into one y), the
    reference-order kernel, and a repeat with a new x, each equal bit for bit to the device path."""
    rng = np.random.default_rng(41)
    cases = [(256, 1024, 1), (4096, 1024, 3), (1024, 4096, 16), (8192, 1024, 70), (512, 2048, 4), (2048, 4096, 1)]
    old_mode = host_mode(rt, mode)
    try:
        staging_cases(rt, rng, cases)
    finally:
        restore_host_mode(rt, old_mode)


def staging_cases(rt, rng, cases):
    for rows, cols, t in cases:
        q8 = synth.q8_rows(rng, rows, cols)
        w = rt.upload(q8, rows, cols)
        try:
            for exact in (False, True) if t <= 4 else (False,):
                old = rt.set_exact(exact)
                try:
                    for rep in range(3):
                        x = synth.x_f32(rng, t, cols)
                        Y = np.full((t, rows), np.nan, np.float32)
                        if t == 1:
                            rt.gemv(w, rows, cols, x[0], Y[0])
                        else:
                            rt.gemm(w, rows, cols, x, t, Y)
                        say("host staging", rows, cols, t, "exact" if exact else "fast", rep)
                        assert np.array_equal(Y.view(np.uint32), gpu_gemm(rt, q8, rows, cols, x, exact=exact, w=w).view(np.uint32))
                finally:
                    rt.set_exact(old)
        finally:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


def random_cases(n=28, seed=2024):
    """Seeded shapes across every product path: rows a multiple of 16 (one tile to 1536 rows), cols a
    multiple of 32 (odd block counts included), t from 1 to 70 (decode, x-resident, streaming, more
    than 64 tokens), normal or heavy-tailed scales."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        rows = 16 * int(rng.integers(1, 97))
        cols = 32 * int(rng.integers(1, 129))
        t = int(rng.choice([1, 2, 3, 4, 5, 7, 9, 12, 16, 17, 23, 32, 33, 40, 47, 64, 65, 70]))
        out.append((i, rows, cols, t, "lognormal" if i % 3 == 2 else "normal"))
    return out


@pytest.mark.parametrize("case", random_cases(), ids=lambda c: f"{c[1]}x{c[2]}t{c[3]}")
def test_random_shapes_every_path(rt, oracle, case):
    """The fast kernels against the F64 closed form at the parity bar, and the reference-order kernel
    against the oracle bit for bit, on seeded random shapes."""
    i, rows, cols, t, dist = case
    q8, x = synth.case(9000 + i, rows, cols, t, dist)
    say("random", rows, cols, t, dist)
    w = rt.upload(q8, rows, cols)
    try:
        got = gpu_gemm(rt, q8, rows, cols, x, w=w)
        assert_parity(got, oracle.gemm_f64(q8, rows, cols, x), f"{rows}x{cols} t={t} {dist}")
        if rows * cols * t <= 1 << 24:
            ex = gpu_gemm(rt, q8, rows, cols, x, exact=True, w=w)
            assert np.array_equal(ex.view(np.uint32), oracle.gemm(q8, rows, cols, x).view(np.uint32))
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


def random_round_cases(n=14, seed=4242):
    """Seeded rounds: 2 to 8 products sharing x, rows 16..1536 and K 32..4096 columns at random, every
    third case of one shape (two products of one shape run as a pair at 5..16 tokens, and at 33..64
    where the plan takes 12 waves), at 1 to 70 tokens (decode rounds, x-resident, streaming, and
    64-token chunks with a short last one)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        k = 2 if i % 3 == 0 else int(rng.integers(2, 9))
        cols = 32 * int(rng.integers(1, 129))
        rows = [16 * int(rng.integers(1, 97)) for _ in range(k)]
        if i % 3 == 0:  # one shape: the pair kernels at 5..16 and 33..64 tokens
            rows = [rows[0]] * k
            t = int(rng.choice([5, 9, 16, 33, 40, 47, 48, 64, 66]))
        else:
            t = int(rng.choice([1, 3, 4, 5, 8, 13, 16, 17, 29, 40, 64, 66, 70]))
        out.append((i, tuple(rows), cols, t))
    return out


@pytest.mark.parametrize("case", random_round_cases(), ids=lambda c: f"{len(c[1])}x{c[1][0]}x{c[2]}t{c[3]}")
def test_random_rounds_equal_singles(rt, oracle, case):
    """rt_gemv_round_dev on seeded random rounds: every product's y has the bits of its own
    rt_gemm_dev at every token count (one launch for the products, a pair for two of one shape,
    the decode round below 5 tokens) and meets the parity bar against F64."""
    i, shapes, cols, t = case
    n = len(shapes)
    rng = np.random.default_rng(9500 + i)
    mats = [synth.q8_rows(rng, r, cols) for r in shapes]
    x = synth.x_f32(rng, t, cols)
    say("random round", shapes, cols, t)
    ws = [rt.upload(m, r, cols) for m, r in zip(mats, shapes)]
    try:
        singles = [gpu_gemm(rt, m, r, cols, x, w=w) for m, r, w in zip(mats, shapes, ws)]
        with Dev(rt) as d:
            dx = d.put(x)
            ys = [d.empty(4 * t * r) for r in shapes]
            W, R, Y = (c.c_void_p * n)(*ws), (c.c_long * n)(*shapes), (c.c_void_p * n)(*ys)
            rt.lib.rt_gemv_round_dev(rt.R, n, W, R, cols, c.c_void_p(dx), cols, t, Y)
            got = [d.get(p, (t, r), np.float32) for p, r in zip(ys, shapes)]
        for g, s1, m, r in zip(got, singles, mats, shapes):
            assert np.array_equal(g.view(np.uint32), s1.view(np.uint32)), r
            assert_parity(g, oracle.gemm_f64(m, r, cols, x), f"round {r}x{cols} t={t}")
    finally:
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))


INVARIANT_CASES = [(256, 1024, 1), (512, 2048, 3), (1024, 4096, 16), (768, 1056, 9), (512, 4096, 40)]


@pytest.mark.parametrize("rows,cols,t", INVARIANT_CASES)
def test_one_hot_x_reads_a_column(rt, rows, cols, t):
    """x = e_j (token k's j differs per token: block edges, the last column) gives column j of d*q
    exactly on the fast kernels: every other term is an exact zero, and x = 1 has no lower limbs on
    the matrix cores. Decode (t <= 4), x-resident (5..16, 1056 columns: half a final pair) and
    streaming (t > 16) kernels."""
    rng = np.random.default_rng(rows + cols + t)
    q8 = synth.q8_rows(rng, rows, cols)
    q, d = synth.split(q8, rows, cols)
    cols_hot = [(31 + 32 * 5 * k + 7 * k) % cols for k in range(t)]
    cols_hot[-1] = cols - 1
    x = np.zeros((t, cols), np.float32)
    for k, j in enumerate(cols_hot):
        x[k, j] = 1.0
    got = gpu_gemm(rt, q8, rows, cols, x)
    want = np.stack([d[:, j // 32].astype(np.float32) * q[:, j].astype(np.float32) for j in cols_hot])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,cols,t", INVARIANT_CASES)
def test_permuting_row_groups_permutes_y(rt, rows, cols, t):
    """Reordering the 16-row groups of W reorders Y the same way, bit for bit: no kernel's per-row
    arithmetic depends on where the row sits."""
    rng = np.random.default_rng(7 * rows + cols + t)
    q8 = synth.q8_rows(rng, rows, cols)
    x = synth.x_f32(rng, t, cols)
    perm = rng.permutation(rows // 16)
    rows_of = (perm[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)
    q8p = q8.reshape(rows, -1)[rows_of].reshape(-1)
    y = gpu_gemm(rt, q8, rows, cols, x)
    yp = gpu_gemm(rt, q8p, rows, cols, x)
    assert np.array_equal(yp.view(np.uint32), y[:, rows_of].view(np.uint32))


@pytest.mark.parametrize("t", [2, 4, 16, 40])
def test_non_finite_x_gives_the_references_classes(rt, oracle, t):
    """An infinity or a NaN in x (token 0: +inf at one column, token 1: NaN at another, the last token
    for t > 2: -inf at the last column) gives, output by output, the class the reference's F32 order
    gives (oracle): NaN where the column's q or d is zero or x holds a NaN, an infinity with the sign
    of q * d otherwise. The other tokens hold the parity bar; the reference-order kernel equals the
    oracle bit for bit. Decode kernel (t <= 4), x-resident (16) and streaming (40) matrix cores,
    whose three-limb split keeps an infinite x whole."""
    rows, cols = 512, 4096
    rng = np.random.default_rng(11 + t)
    q8 = synth.q8_rows(rng, rows, cols)
    x = synth.x_f32(rng, t, cols)
    x[0, 77] = np.inf
    x[1, 1000] = np.nan
    bad = [0, 1]
    if t > 2:
        x[t - 1, cols - 1] = -np.inf
        bad.append(t - 1)
    say("non-finite x", t)
    ref = oracle.gemm(q8, rows, cols, x)
    got = gpu_gemm(rt, q8, rows, cols, x)
    for k in bad:
        assert not np.isfinite(ref[k]).any()
        for cls in (np.isnan, np.isposinf, np.isneginf):
            assert np.array_equal(cls(got[k]), cls(ref[k])), f"token {k}: {cls.__name__}"
    good = [k for k in range(t) if k not in bad]
    if good:
        assert_parity(got[good], oracle.gemm_f64(q8, rows, cols, x[good]), f"finite tokens t={t}")
    ex = gpu_gemm(rt, q8, rows, cols, x, exact=True)
    assert np.array_equal(ex, ref, equal_nan=True)


def test_edge_scales(rt, oracle):
    """Zero scales give +0; subnormal, largest-finite and negative binary16 scales; q at -128..127 (the
    GGUF byte range, wider than the generator's)."""
    rows, cols = 64, 1024
    rng = np.random.default_rng(5)
    q = rng.integers(-128, 128, size=(rows, cols), dtype=np.int8)
    d = np.zeros((rows, cols // 32), np.float16)
    d[16:32] = np.float16(6.0e-8)  # the smallest subnormal
    d[32:48] = rng.integers(1, 1024, size=(16, cols // 32)).astype(np.uint16).view(np.float16)  # every subnormal class
    d[48:64] = -np.float16(65504.0) / np.float16(1 << 14)
    q8 = synth.join(q, d)
    x = synth.x_f32(rng, 2, cols)
    want = oracle.gemm_f64(q8, rows, cols, x)
    for exact in (False, True):
        got = gpu_gemm(rt, q8, rows, cols, x, exact=exact)
        assert np.all(got[:, :16].view(np.uint32) == 0)
        assert_parity(got[:, 16:], want[:, 16:], f"edge scales exact={exact}")
    ex = gpu_gemm(rt, q8, rows, cols, x, exact=True)
    assert np.array_equal(ex.view(np.uint32), oracle.gemm(q8, rows, cols, x).view(np.uint32))


def test_fill_generator(rt):
    """rt_q8_fill_dev: q in [-127, 127], roughly uniform; d = |N(0, 0.02)|/127 in binary16; the bytes
    are a function of the seed."""
    rows, cols = 1024, 4096
    with Dev(rt) as d:
        p = d.empty(rows * cols // 32 * 34)
        rt.lib.rt_q8_fill_dev(rt.R, c.c_void_p(p), rows, cols, 7, 0, 0.0, 0.02)
        a = d.get(p, rows * cols // 32 * 34, np.uint8)
        rt.lib.rt_q8_fill_dev(rt.R, c.c_void_p(p), rows, cols, 7, 0, 0.0, 0.02)
        b = d.get(p, rows * cols // 32 * 34, np.uint8)
    assert np.array_equal(a, b)
    q, dd = synth.split(a, rows, cols)
    assert q.min() == -127 and q.max() == 127
    assert abs(q.astype(np.float64).mean()) < 0.1
    df = dd.astype(np.float64)
    assert np.all(np.isfinite(df)) and np.all(df >= 0)
    assert abs(df.mean() / (0.02 * np.sqrt(2 / np.pi) / 127) - 1) < 0.01


def test_c_drop_in_caller(tmp_path):
    """tests/c/drop_in.c, a C program written against include/q8_rt.h and include/q8_gguf.h alone,
    passes its checks."""
    exe = tmp_path / "drop_in"
    lib_dir = os.path.join(ROOT, "intel-phi-apl_amd")
    subprocess.run(["gcc", "-std=gnu11", "-O2", "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "c", "drop_in.c"), "-L", lib_dir,
                    "-lq8rt", "-Wl,-rpath," + lib_dir, "-lm", "-o", str(exe)], check=True)
    p = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    say(p.stdout)
    assert p.returncode == 0, p.stdout + p.stderr


def _kernels_launched(rt, fn):
    """(name, grid threads) of the first kernel of every product fn makes, from the runtime's own
    kernel records (rt_ktime)."""
    n = 64
    rt.lib.rt_ktime(rt.R, 1)
    try:
        fn()
        arrs = [np.zeros(n, np.int32), np.zeros(n, np.int64), np.zeros(n, np.int64), np.zeros(n, np.int64), np.zeros(n, np.float32)]
        names, grid = c.create_string_buffer(64 * n), np.zeros(n, np.int64)
        got = rt.lib.rt_ktime_read(rt.R, *(a.ctypes.data_as(c.c_void_p) for a in arrs), names, grid.ctypes.data_as(c.c_void_p), n)
    finally:
        rt.lib.rt_ktime(rt.R, 0)
    return [(names.raw[64 * i:64 * i + 64].split(b"\0")[0].decode(), int(grid[i])) for i in range(got)]


def _targs(name):
    return [int(v) for v in name.split("<")[1].rstrip(">").split(",")]


@pytest.mark.parametrize("rows,cols,pair,t", [(4096, 4096, False, 1), (4096, 12288, False, 1), (12288, 4096, True, 1), (151936, 4096, False, 1),
                                              (3072, 2048, False, 1), (12288, 4096, True, 3), (4096, 12288, False, 4), (12288, 4096, False, 16),
                                              (4096, 12288, False, 16), (6144, 4096, False, 8)])
def test_read_floor_runs_on_the_products_grid(rt, rows, cols, pair, t):
    """The floor the benchmark holds a product against is that product's own grid: rt_q8_read_dev
    launches the read twin of the kernel the product launches (read_k<RW, NW, PAIR, MT> for
    gemv_k<MT, RW, S, NW, PAIR>, read_xres<KP, NW, SC> for gemm_xres<KP, NW, SC>) with the same
    number of threads, as the runtime's kernel records show."""
    rng = np.random.default_rng(rows + cols + t)
    mats = [synth.q8_rows(rng, rows, cols) for _ in range(2 if pair else 1)]
    ws = [rt.upload(q8, rows, cols) for q8 in mats]
    V = c.c_void_p
    try:
        with Dev(rt) as d:
            dx, dy, sink = d.put(np.zeros(t * cols, np.float32)), d.empty(4 * t * rows), d.put(np.zeros(rows, np.uint32))
            if pair:
                prod = lambda: rt.lib.rt_gemv_swiglu_dev(rt.R, V(ws[0]), V(ws[1]), rows, cols, V(dx), cols, t, V(dy))  # noqa: E731
            else:
                prod = lambda: rt.lib.rt_gemm_dev(rt.R, V(ws[0]), rows, cols, V(dx), cols, t, V(dy))  # noqa: E731
            (pk, pg), = _kernels_launched(rt, prod)
            (fk, fg), = _kernels_launched(rt, lambda: rt.lib.rt_q8_read_dev(rt.R, V(ws[0]), V(ws[1]) if pair else None, rows, cols, V(dx), cols, t,
                                                                             V(sink)))
    finally:
        for w in ws:
            rt.lib.rt_q8_free(rt.R, V(w))
    say("product", pk, pg, "floor", fk, fg)
    assert fg == pg
    if t <= 4:
        mt, rw, s, nw, p = _targs(pk)
        assert pk.startswith("gemv_k<") and fk == f"read_k<{rw}, {nw}, {p}, {mt}>" and s == 1
    else:
        assert pk.startswith("gemm_xres<") and fk == pk.replace("gemm_xres", "read_xres")


@pytest.mark.parametrize("rows,cols,pair,t", [(4096, 4096, False, 1), (6144, 4096, False, 1), (4096, 12288, False, 1), (12288, 4096, True, 1),
                                              (3072, 2048, False, 1), (6144, 2048, True, 1), (2048, 6144, False, 1), (151936, 4096, False, 1),
                                              (12288, 4096, True, 2), (12288, 4096, True, 4), (4096, 12288, False, 3),
                                              (12288, 4096, False, 16), (4096, 12288, False, 16), (48, 4096, False, 5), (1888, 512, False, 9),
                                              (64, 1056, False, 7)])
def test_read_floor_checksum(rt, rows, cols, pair, t):
    """rt_q8_read_dev (the product's loads on its grid at t tokens, no arithmetic: the floor the
    benchmark sets each product against) reads every byte of the matrix or matrices: its wrapping
    sum of the 32-bit words read equals numpy's, with x = 0. At 1 to 4 tokens (the decode kernel)
    each scale is read by two lanes; at 5 to 16 (the x-resident matrix-core kernel, its K split)
    each weight word and scale is added once, on partial row tiles (48, 1888 rows) and with a
    block count that leaves half a pair (1056 columns, 33 blocks) too."""
    rng = np.random.default_rng(rows + cols + pair + 10 * t)
    mats = [synth.q8_rows(rng, rows, cols) for _ in range(2 if pair else 1)]
    want = 0
    for q8 in mats:
        blk = q8.reshape(-1, 34)
        want += int(blk[:, 2:].copy().view(np.uint32).astype(np.uint64).sum()) + (2 if t <= 4 else 1) * int(blk[:, :2].copy().view(np.uint16).astype(np.uint64).sum())
    ws = [rt.upload(q8, rows, cols) for q8 in mats]
    try:
        with Dev(rt) as d:
            dx, sink = d.put(np.zeros(t * cols, np.float32)), d.put(np.zeros(rows, np.uint32))
            rt.lib.rt_q8_read_dev(rt.R, c.c_void_p(ws[0]), c.c_void_p(ws[1]) if pair else None, rows, cols, c.c_void_p(dx), cols, t,
                                  c.c_void_p(sink))
            got = d.get(sink, (rows,), np.uint32)
    finally:
        for w in ws:
            rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
    assert int(got.astype(np.uint64).sum()) % 2**32 == want % 2**32
