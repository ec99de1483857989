"""The oracle pinned: against the reference's golden gate files, its compiled sources, fixtures made
from them, exact rational arithmetic and invariants. CPU only."""
import hashlib
import os
from fractions import Fraction

import numpy as np
import pytest

import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden_lines(name):
    return [l.split() for l in open(os.path.join(GOLDEN, name)).read().splitlines() if l.strip()]


def test_gate_a_fma(oracle):
    """fmaf's single rounding on the reference's gate A inputs (tests/golden/gate-a.txt:1)."""
    (line,) = golden_lines("gate-a.txt")
    h, c0, c1, clast = oracle.gate_a()
    assert line == ["n", "4096", "hash", f"{h:016x}", "c0", f"{c0:08x}", "c1", f"{c1:08x}", "clast", f"{clast:08x}"]


def test_gate21_conversions(oracle):
    """int8, uint8, binary16 (all 65536 patterns) and the 16-lane tree, the reference's gate 2.1
    golden hashes (tests/golden/gate-2.1.txt:1-7), in file order."""
    got = oracle.gate21()
    want = golden_lines("gate-2.1.txt")
    assert [w[0] for w in want] == ["s8", "u8fma", "u8mul", "b16", "bcast", "f16", "hsum"]
    assert [f"{g:016x}" for g in got] == [w[4] for w in want]


def test_half_exhaustive(oracle):
    """binary16 -> binary32 for all 65536 patterns against numpy's conversion (exact): non-NaN bit
    for bit, NaN to NaN with the same sign and payload (t_knc_half.c:19-40)."""
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([oracle.half(v) for v in range(65536)], np.float32).view(np.uint32)
    nan = ((h >> 10) & 31 == 31) & (h & 1023 != 0)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.array_equal(got[nan] & ~np.uint32(0x00400000), want[nan] & ~np.uint32(0x00400000))


def load_fixtures():
    z = np.load(os.path.join(GOLDEN, "ref_products.npz"))
    cases = []
    for i in range(int(z["ncases"][0])):
        seed, rows, cols, t, logn = (int(v) for v in z[f"c{i}_meta"])
        cases.append((seed, rows, cols, t, logn, z[f"c{i}_q8"], z[f"c{i}_x"], z[f"c{i}_y"]))
    return z, cases


def test_fixture_inputs_regenerate():
    """The fixtures' inputs are what tests/synth.py draws from their seeds (so the GPU tests can use
    either)."""
    z, cases = load_fixtures()
    for seed, rows, cols, t, logn, q8, x, _ in cases:
        q8b, xb = synth.case(seed, rows, cols, t, "lognormal" if logn else "normal")
        assert np.array_equal(q8, q8b) and np.array_equal(x, xb)
    q8, x = synth.case(0, 4096, 4096, 1)
    assert hashlib.sha256(q8.tobytes()).digest() == z["cfg1_sha_q8"].tobytes()
    assert hashlib.sha256(x.tobytes()).digest() == z["cfg1_sha_x"].tobytes()


def test_oracle_matches_reference_fixtures(oracle):
    """Bit for bit against the reference's compiled gemv/gemm outputs (tests/golden/ref_products.npz)."""
    z, cases = load_fixtures()
    for seed, rows, cols, t, logn, q8, x, y in cases:
        got = oracle.gemm(q8, rows, cols, x)
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), (seed, rows, cols, t)
        got_mt = oracle.gemm(q8, rows, cols, x, threads=3)
        assert np.array_equal(got_mt.view(np.uint32), y.view(np.uint32))
    q8, x = synth.case(0, 4096, 4096, 1)
    assert np.array_equal(oracle.gemm(q8, 4096, 4096, x)[0].view(np.uint32), z["cfg1_y"].view(np.uint32))


@pytest.mark.parametrize("rows,cols,t", [(16, 512, 1), (16, 512, 2), (64, 512, 3), (512, 512, 4), (1888, 512, 5), (16, 512, 6), (16, 512, 7),
                                         (64, 512, 8), (16, 512, 9), (16, 512, 15), (512, 512, 16), (16, 512, 17), (64, 512, 40), (32, 4096, 2)])
def test_oracle_matches_compiled_reference(oracle, reference, rows, cols, t):
    """Against the reference's gemm_i_thread / gemv_i_thread built from its sources, the shapes of its
    own gemm == gemv gate (scripts/check.sh:132-149)."""
    if reference is None:
        pytest.skip("oracle/_ref not built (the reference's sources are not in this container)")
    q8, x = synth.case(1000 + rows + t, rows, cols, t)
    y_ref = reference.gemm(q8, rows, cols, x)
    assert np.array_equal(oracle.gemm(q8, rows, cols, x).view(np.uint32), y_ref.view(np.uint32))
    assert np.array_equal(reference.gemv(q8, rows, cols, x[0]).view(np.uint32), y_ref[0].view(np.uint32))


def test_f64_closed_form_exact_rationals(oracle):
    """The F64 closed form against exact rational arithmetic on tiny shapes: every term d*q*x is exact
    in F64 and the sum of 64 of them differs from the exact sum by at most 64 ulp."""
    for seed in range(4):
        rows, cols = 16, 64
        q8, x = synth.case(50 + seed, rows, cols, 1)
        q, d = synth.split(q8, rows, cols)
        got = oracle.gemm_f64(q8, rows, cols, x)[0]
        for r in range(rows):
            exact = sum(Fraction(float(d[r, k // 32])) * int(q[r, k]) * Fraction(float(x[0, k])) for k in range(cols))
            assert abs(Fraction(got[r]) - exact) <= abs(exact) * Fraction(64, 2**53) + Fraction(1, 2**1000)


def test_f32_order_close_to_f64(oracle):
    """The reference's F32 order stays within F32 rounding of the closed form (config 1's shape)."""
    from parity import metrics

    q8, x = synth.case(0, 4096, 4096, 1)
    m = metrics(oracle.gemm(q8, 4096, 4096, x), oracle.gemm_f64(q8, 4096, 4096, x))
    assert m["nrmse"] < 1e-6 and m["max_rel"] < 2e-5, m


def test_invariants(oracle):
    """x = e_j gives column j of d*q exactly; zero scales give +0; permuting 16-row groups permutes y;
    a prefix of groups is the product of those rows."""
    rows, cols = 64, 256
    q8, x = synth.case(77, rows, cols, 1)
    q, d = synth.split(q8, rows, cols)
    for j in (0, 31, 32, 255):
        e = np.zeros(cols, np.float32)
        e[j] = 1.0
        col = oracle.gemm(q8, rows, cols, e)[0]
        assert np.array_equal(col, (d[:, j // 32].astype(np.float32) * q[:, j].astype(np.float32)))
    z = synth.join(q, np.zeros_like(d))
    y0 = oracle.gemm(z, rows, cols, x)[0]
    assert np.all(y0.view(np.uint32) == 0)
    y = oracle.gemm(q8, rows, cols, x)[0]
    perm = np.array([2, 0, 3, 1])
    qp = q.reshape(4, 16, cols)[perm].reshape(rows, cols)
    dp = d.reshape(4, 16, cols // 32)[perm].reshape(rows, cols // 32)
    yp = oracle.gemm(synth.join(qp, dp), rows, cols, x)[0]
    assert np.array_equal(yp, y.reshape(4, 16)[perm].reshape(-1))
    assert np.array_equal(oracle.gemm(q8[: 32 * cols // 32 * 34], 32, cols, x)[0], y[:32])


def test_linearity_f64(oracle):
    rows, cols = 32, 512
    q8, x = synth.case(5, rows, cols, 2)
    a, b = 0.75, -2.5
    xc = (a * x[0].astype(np.float64) + b * x[1].astype(np.float64)).astype(np.float32)
    y = oracle.gemm_f64(q8, rows, cols, x)
    yc = oracle.gemm_f64(q8, rows, cols, xc)[0]
    # xc is rounded to F32: compare with the F64 product of the rounded input's linear parts
    assert np.allclose(yc, a * y[0] + b * y[1], rtol=1e-6, atol=1e-6 * np.abs(y).max())


def test_repack_s_definition(oracle):
    """Form S byte by byte against an independent index formula."""
    rows, cols = 48, 96
    q8, _ = synth.case(9, rows, cols, 1)
    q, d = synth.split(q8, rows, cols)
    got = oracle.repack_s(q8, rows, cols)
    want = np.concatenate([np.concatenate([q[16 * g:16 * g + 16].view(np.uint8).ravel(), d[16 * g:16 * g + 16].view(np.uint8).ravel()])
                           for g in range(rows // 16)])
    assert np.array_equal(got, want)


def test_planted_mistakes_are_caught(oracle):
    """The checks have teeth: plausible slips in an F32 product (one term dropped, the scale of a
    neighbouring block, a transposed operand, a sign) each fail the parity bar against the F64 form."""
    from parity import metrics

    rows, cols = 64, 512
    q8, x = synth.case(21, rows, cols, 1)
    q, d = synth.split(q8, rows, cols)
    ref = oracle.gemm_f64(q8, rows, cols, x)[0]
    qf, df, xf = q.astype(np.float64), np.repeat(d.astype(np.float64), 32, axis=1), x[0].astype(np.float64)

    def fails(y):
        m = metrics(y, ref)
        return m["nrmse"] > 1e-5 or m["max_rel"] > 1e-4

    assert not fails((qf * df) @ xf)
    dropped = qf.copy()
    dropped[:, 100] = 0
    assert fails((dropped * df) @ xf)
    assert fails((qf * np.roll(df, 32, axis=1)) @ xf)
    assert fails((qf * df)[:, ::-1] @ xf)
    assert fails((-qf * df) @ xf)


def _logits(rng, n):
    return rng.standard_normal(n).astype(np.float32) * 4


def test_next_token_matches_reference(oracle, reference):
    """q8o_next against the reference's rt_maxv + rt_index_of, and numpy: ragged lengths, ties (the
    lowest index wins), NaN entries (fmaxf skips them), all-negative and constant arrays."""
    if reference is None:
        pytest.skip("the reference's sources are not here to build oracle/_ref")
    rng = np.random.default_rng(11)
    cases = []
    for n in (1, 2, 15, 16, 17, 31, 1000, 4096, 4097, 151936):
        a = _logits(rng, n)
        cases.append(a)
        t = a.copy()
        j = rng.integers(0, n, 3)
        t[j] = t.max() + 1.0  # a three-way tie at the top
        cases.append(t)
        if n > 2:
            u = a.copy()
            u[rng.integers(0, n, max(1, n // 10))] = np.nan
            u[0] = np.nan
            cases.append(u)
    cases += [np.full(33, -3.0, np.float32), -np.abs(_logits(rng, 100)) - 1]
    for a in cases:
        got = oracle.next(a)
        assert got == reference.next(a), (a.size, got, reference.next(a))
        if not np.isnan(a).all():
            assert got == int(np.nanargmax(a))


def test_row_read_matches_reference(oracle, reference):
    """q8o_row equals the reference's rt_q8_row on form I bit for bit, and numpy's d * q (exact)."""
    rows, cols = 64, 512
    q8, _ = synth.case(44, rows, cols, 1, "lognormal")
    q, d = synth.split(q8, rows, cols)
    for r in (0, 1, 15, 16, 37, 63):
        got = oracle.row(q8, cols, r)
        want = np.repeat(d[r].astype(np.float32), 32) * q[r].astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        if reference is not None:
            assert np.array_equal(got.view(np.uint32), reference.row(q8, rows, cols, r).view(np.uint32))


def test_rmsnorm_f64_matches_reference_f32(oracle, reference):
    """q8o_rmsnorm_f64 against the reference's own F32 norm, composed from its host rt_sum, rt_s_div,
    rt_s_add and rt_s_rsqrt (oracle/_ref): F32 error only (<= 1e-6 of the largest output), on
    lengths that are and are not whole 16-lane blocks, with and without eps."""
    if reference is None:
        pytest.skip("oracle/_ref is not built")
    rng = np.random.default_rng(41)
    for cols in (1024, 4096, 2064, 100):
        x = (3 * rng.standard_normal(cols)).astype(np.float32)
        nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
        for eps in (1e-6, 1e-5, 0.0):
            f64 = oracle.rmsnorm_f64(x[None], nw, eps)[0]
            r32 = reference.rmsnorm_f32(x, nw, eps)
            assert np.max(np.abs(f64 - r32)) <= 1e-6 * np.max(np.abs(f64)), (cols, eps)


def test_rmsnorm_f64_closed_forms(oracle):
    """A constant vector's norm in closed form; at eps = 0, scaling x by a power of two changes
    nothing (exactly) and the normed x has unit RMS; nw multiplies elementwise."""
    cols = 256
    ones = np.ones(cols, np.float32)
    for cval in (2.0, -0.5, 1e-3, 7.25):
        x = np.full((1, cols), cval, np.float32)
        got = oracle.rmsnorm_f64(x, ones, 1e-6)[0]
        want = float(np.float32(cval)) / np.sqrt(1e-6 + float(np.float32(cval)) ** 2)
        assert np.allclose(got, want, rtol=1e-13, atol=0), cval  # a 256-term F64 sum: ~1e-14
    rng = np.random.default_rng(42)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    a = oracle.rmsnorm_f64(x, ones, 0.0)
    assert np.array_equal(a, oracle.rmsnorm_f64(x * np.float32(4.0), ones, 0.0))
    assert np.allclose(np.mean(a * a, axis=1), 1.0, rtol=1e-13, atol=0)
    nw = rng.standard_normal(cols).astype(np.float32)
    assert np.array_equal(oracle.rmsnorm_f64(x, nw, 1e-5), nw.astype(np.float64) * oracle.rmsnorm_f64(x, ones, 1e-5))


def test_gemm_f64d_is_gemm_f64_on_f32_x(oracle):
    """The F64-x product equals the F32-x one where x is an F32 vector, and is linear in x."""
    rows, cols = 48, 256
    q8, x = synth.case(43, rows, cols, 3)
    assert np.array_equal(oracle.gemm_f64d(q8, rows, cols, x.astype(np.float64)), oracle.gemm_f64(q8, rows, cols, x))
    rng = np.random.default_rng(44)
    x1, x2 = rng.standard_normal((2, cols))
    lhs = oracle.gemm_f64d(q8, rows, cols, 0.75 * x1 + x2)
    rhs = 0.75 * oracle.gemm_f64d(q8, rows, cols, x1) + oracle.gemm_f64d(q8, rows, cols, x2)
    assert np.allclose(lhs, rhs, rtol=1e-12, atol=1e-12)


def swiglu_violations(f):
    """The facts the mathematics fixes for the reference's FFN activation, Sig = {1 / (1 + exp(min(700,
    -g)))} and SiLU = {g x Sig g}, times u (src/apl/qwen35.apl:37-38, 124-126), checked on f(g, u) (F64
    arrays in, F64 out). Returns the names of the facts f breaks; the oracle must break none."""
    bad = []
    rng = np.random.default_rng(51)
    g = rng.uniform(-30.0, 30.0, 4000)
    u = rng.uniform(-4.0, 4.0, 4000)
    ones = np.ones_like(g)
    if not np.all(f(np.zeros(8), np.linspace(-3, 3, 8)) == 0.0):
        bad.append("SiLU(0) u = 0")
    # SiLU(g) - SiLU(-g) = g (1 / (1 + e^-g) + 1 / (1 + e^g)) = g: pins the exponent's sign
    if not np.allclose(f(g, ones) - f(-g, ones), g, rtol=1e-12, atol=1e-12):
        bad.append("SiLU(g) - SiLU(-g) = g")
    # Sig(ln 3) = 1 / (1 + 1/3) = 3/4 exactly in the reals
    l3 = np.log(3.0)
    if not np.allclose(f(np.full(6, l3), u[:6]), 0.75 * l3 * u[:6], rtol=1e-14, atol=0):
        bad.append("SiLU(ln 3) u = 3/4 ln 3 u")
    # a large positive g: Sig -> 1, the output is g u
    big = np.array([40.0, 60.0, 100.0, 700.0, 1e4])
    if not np.allclose(f(big, np.full(5, -1.5)), -1.5 * big, rtol=1e-15, atol=0):
        bad.append("SiLU(g) u = g u for large g")
    # through the 700 clamp: -800 and -1e6 give exp(700), finite, so the output is a finite ~0
    neg = np.array([-800.0, -1e6, -709.0, -701.0])
    y = f(neg, np.full(4, 2.0))
    if not (np.all(np.isfinite(y)) and np.all(np.abs(y) < 1e-290)):
        bad.append("finite ~0 through the 700 clamp")
    # linear in u
    if not np.allclose(f(g, 3.0 * u), 3.0 * f(g, u), rtol=1e-14, atol=1e-300):
        bad.append("linear in u")
    # the textbook logistic at a few points: Sig(g) = (1 + tanh(g / 2)) / 2
    pts = np.array([-5.0, -1.0, 0.5, 2.0, 7.0])
    if not np.allclose(f(pts, ones[:5]), pts * (1.0 + np.tanh(pts / 2.0)) / 2.0, rtol=1e-14, atol=1e-300):
        bad.append("Sig(g) = (1 + tanh(g / 2)) / 2")
    return bad


def test_swiglu_f64_pinned(oracle):
    """q8o_swiglu_f64 meets every fact of swiglu_violations; the mistakes one could plant in it (the
    exponent's sign flipped, the x u dropped, the clamp's min turned into max, the logistic's 1 +
    left out) each break at least one."""
    assert swiglu_violations(oracle.swiglu_f64) == []

    planted = {
        "exp(+g)": lambda g, u: g / (1.0 + np.exp(np.minimum(700.0, g))) * u,
        "x u dropped": lambda g, u: g / (1.0 + np.exp(np.minimum(700.0, -g))),
        "max for min": lambda g, u: g / (1.0 + np.exp(np.maximum(700.0, -g))) * u,
        "no 1 +": lambda g, u: g / np.exp(np.minimum(700.0, -g)) * u,
        "u for g": lambda g, u: u / (1.0 + np.exp(np.minimum(700.0, -g))) * u,
    }
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for name, f in planted.items():
            assert swiglu_violations(f), f"the planted mistake '{name}' passes every check"


def test_reference_flag_builds_agree():
    """The reference's host model built with its own flags (-O2 -ffp-contract=off, fmaf a libm call)
    and with -mfma (fmaf inlined) give the same bits: fmaf is correctly rounded either way. Both are
    timed as the CPU baseline."""
    from oracle_ffi import ORACLE_DIR, Reference

    paths = [os.path.join(ORACLE_DIR, "_ref", n) for n in ("libref.so", "libref_flags.so")]
    if not all(os.path.exists(p) for p in paths):
        pytest.skip("oracle/_ref is not built")
    a, b = Reference(paths[0]), Reference(paths[1])
    for seed, rows, cols, t in [(61, 64, 512, 1), (62, 48, 1024, 5), (63, 128, 256, 17)]:
        q8, x = synth.case(seed, rows, cols, t, "lognormal" if seed % 2 else "normal")
        ya, yb = a.gemm(q8, rows, cols, x), b.gemm(q8, rows, cols, x)
        assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), (rows, cols, t)
