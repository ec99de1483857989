"""GPU parity at the output head and the draft head, and the batch deviation of the fast kernels.

  - Logits (src/apl/qwen35.apl:158-160): the 151936 x 4096 output head at 1, 3 and 16 tokens, the
    fast kernels against the F64 closed form at the parity bar, the reference-order kernel against
    the oracle's F32 order bit for bit (1 and 3 tokens);
  - DraftLogits (qwen35.apl:170-172): the first 32768 rows of the same handle equal the first
    32768 outputs of the full product bit for bit;
  - the 9B model's own 248320 x 4096 output matrix (ref_harness.apl:82-83) at 1 and 4 tokens;
  - the reference keeps gemm(t)[k] == gemv(x[k]) bit for bit (src/card/gemm.h:7). Here the
    reference-order kernel keeps it, the decode kernel (t <= 4) keeps it, and the matrix-core
    product (t >= 5, any K split) does not: its outputs differ from the one-token product's by the
    F32 rounding of another summation order, bounded here by the parity bar;
  - the reference's own gemm gate (scripts/check.sh:132-149) on its shapes and token counts, in the
    reference-order kernel.
"""
import ctypes as c
import os

import numpy as np
import pytest

from parity import assert_parity, metrics

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN, DRAFT = 151936, 4096, 32768
# the token counts of the reference's gemm gate (scripts/check.sh:132-149), which crosses every
# token chunk of its gemm (src/card/gemm.c)
GATE_T = (1, 2, 3, 4, 5, 6, 7, 8, 9, 15, 16, 17, 40)


def say(*a):
    print(*a, flush=True)


class Handle:
    """A Q8_0 matrix drawn on the device (rt_q8_fill_dev), repacked into a buffer that becomes a
    registered handle (rt_q8_repack_dev); its GGUF rows also on the host, for the oracle."""

    def __init__(self, rt, rows, cols, seed, dist=0, mu=0.0, sigma=0.02):
        self.rt, self.rows, self.cols = rt, rows, cols
        nbytes = rows * cols // 32 * 34
        src = rt.alloc(nbytes)
        rt.lib.rt_q8_fill_dev(rt.R, c.c_void_p(src), rows, cols, seed, dist, c.c_float(mu), c.c_float(sigma))
        self.q8 = np.empty(nbytes, np.uint8)
        rt.from_dev(self.q8, src)
        self.w = rt.alloc(nbytes)
        rt.lib.rt_q8_repack_dev(rt.R, c.c_void_p(src), rows, cols, c.c_void_p(self.w))
        rt.sync()
        rt.free(src)

    def product(self, x, rows=None, exact=False):
        """Y [t rows] = X W[:rows]^T through rt_gemm_dev."""
        rt = self.rt
        rows = rows or self.rows
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.cols)
        t = x.shape[0]
        old = rt.set_exact(exact)
        dx, dy = rt.alloc(x.nbytes), rt.alloc(4 * t * rows)
        try:
            rt.to_dev(dx, x)
            rt.lib.rt_gemm_dev(rt.R, c.c_void_p(self.w), rows, self.cols, c.c_void_p(dx), self.cols, t, c.c_void_p(dy))
            y = np.empty((t, rows), np.float32)
            rt.from_dev(y, dy)
        finally:
            rt.free(dx)
            rt.free(dy)
            rt.set_exact(old)
        return y

    def close(self):
        self.rt.free(self.w)


@pytest.fixture(scope="module")
def head(rt):
    say("head: drawing 151936 x 4096 Q8_0 on the device")
    h = Handle(rt, VOCAB, HIDDEN, seed=151936)
    yield h
    h.close()


@pytest.mark.parametrize("t", [1, 3, 16])
def test_output_head_parity(rt, oracle, head, t):
    """The 151936 x 4096 head: fast kernels at the parity bar against F64, every output finite."""
    x = np.random.default_rng(1000 + t).standard_normal((t, HIDDEN), dtype=np.float32)
    say(f"head t={t}: GPU product")
    y = head.product(x)
    say(f"head t={t}: F64 oracle")
    want = oracle.gemm_f64(head.q8, VOCAB, HIDDEN, x)
    m = assert_parity(y, want, f"head t={t}")
    say(f"head t={t}:", m)


@pytest.mark.parametrize("t", [1, 3])
def test_output_head_reference_order(rt, oracle, head, t):
    """The reference-order kernel on the head equals the oracle's F32 order bit for bit."""
    x = np.random.default_rng(2000 + t).standard_normal((t, HIDDEN), dtype=np.float32)
    y = head.product(x, exact=True)
    want = oracle.gemm(head.q8, VOCAB, HIDDEN, x, threads=8)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", [1, 3])
def test_draft_head_is_prefix(rt, oracle, head, t):
    """rt_gemm_dev with rows = 32768 on the 151936-row handle: the first 32768 outputs of the full
    product, bit for bit, in the fast and the reference-order kernels; and at the parity bar."""
    x = np.random.default_rng(3000 + t).standard_normal((t, HIDDEN), dtype=np.float32)
    for exact in (False, True):
        full = head.product(x, exact=exact)
        draft = head.product(x, rows=DRAFT, exact=exact)
        assert np.array_equal(draft.view(np.uint32), full[:, :DRAFT].view(np.uint32)), f"exact={exact}"
    want = oracle.gemm_f64(head.q8[: DRAFT * HIDDEN // 32 * 34], DRAFT, HIDDEN, x)
    assert_parity(draft, want, f"draft t={t}")


MODEL_VOCAB = 248320  # the 9B model's own output matrix (src/apl/ref_harness.apl:82-83)


@pytest.mark.parametrize("t", [1, 4])
def test_model_head_248320_rows(rt, oracle, t):
    """The 9B model's own output head, 248320 x 4096 (1.08 GB, 31040 workgroups of the decode
    kernel): the fast kernels at the parity bar against F64 at 1 and 4 tokens, every output finite."""
    say("model head: drawing 248320 x 4096 Q8_0 on the device")
    h = Handle(rt, MODEL_VOCAB, HIDDEN, seed=248320 + t)
    try:
        x = np.random.default_rng(4000 + t).standard_normal((t, HIDDEN), dtype=np.float32)
        say(f"model head t={t}: GPU product")
        y = h.product(x)
        say(f"model head t={t}: F64 oracle")
        m = assert_parity(y, oracle.gemm_f64(h.q8, MODEL_VOCAB, HIDDEN, x), f"model head t={t}")
        say(f"model head t={t}:", m)
    finally:
        h.close()


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (4096, 12288)])
def test_batch_deviation_is_bounded(rt, oracle, rows, cols):
    """gemm(t)[k] against gemv(x[k]) (src/card/gemm.h:7): bit for bit in the reference-order kernel at
    the token counts the reference's gate runs (GATE_T) and in the decode kernel at t = 2, 3, 4 (16 rows a workgroup at 2 and 4 tokens on
    4096x12288, 8 at 1 and 3: the rows a workgroup do not change a row's sums); at t >= 5 (the
    matrix-core product) and at every K split tried (1, 3 and the planner's), within the parity bar
    of the one-token product and of F64."""
    h = Handle(rt, rows, cols, seed=rows + cols)
    try:
        X = np.random.default_rng(rows ^ cols).standard_normal((40, cols), dtype=np.float32)
        one = np.concatenate([h.product(X[k]) for k in range(40)])
        one_exact = np.concatenate([h.product(X[k], exact=True) for k in range(40)])
        f64 = oracle.gemm_f64(h.q8, rows, cols, X)
        assert_parity(one, f64, "gemv per token")
        for t in (2, 3, 4):
            y = h.product(X[:t])
            assert np.array_equal(y.view(np.uint32), one[:t].view(np.uint32)), f"decode kernel t={t}"
        for t in GATE_T:
            y = h.product(X[:t], exact=True)
            assert np.array_equal(y.view(np.uint32), one_exact[:t].view(np.uint32)), f"reference order t={t}"
        worst = 0.0
        for ks in (0, 1, 3):
            rt.gemm_force(ks=ks)
            try:
                for t in (3, 4, 5, 16, 17, 40):
                    y = h.product(X[:t])
                    m = assert_parity(y, one[:t], f"t={t} ks={ks or 'planned'} against gemv")
                    assert_parity(y, f64[:t], f"t={t} ks={ks or 'planned'} against F64")
                    worst = max(worst, m["max_rel"])
            finally:
                rt.gemm_force()
        say(f"{rows}x{cols}: largest max-rel between gemm(t)[k] and gemv(x[k]) at t >= 3: {worst:.3e}")
    finally:
        h.close()


MC_T = (5, 16, 17, 40, 64, 65, 70)


@pytest.mark.parametrize("rows,cols", [(12288, 4096), (4096, 12288), (151936, 4096)])
def test_matrix_core_bits_independent_of_t(rt, oracle, rows, cols):
    """On the matrix cores (t >= 5) a token's output has the same bits whatever the number of tokens
    it was computed with: the K split is a function of the matrix's shape alone, and every 64-token
    launch of a longer X, the last one too however few tokens it holds, runs on the matrix cores.
    The 9B FFN shapes (one token tile on the x-resident kernel, two to four on the streaming one) and
    the output head (whose K split the workspace limits); 65 tokens end in a one-token launch."""
    h = Handle(rt, rows, cols, seed=3 * rows + cols)
    head = rows == VOCAB
    try:
        n = 17 if head else max(MC_T)
        X = np.random.default_rng(rows + 2 * cols).standard_normal((n, cols), dtype=np.float32)
        full = h.product(X)
        for t in MC_T:
            if t > n:
                continue
            say(f"{rows}x{cols} t={t} against t={n}")
            y = h.product(X[:t])
            assert np.array_equal(y.view(np.uint32), full[:t].view(np.uint32)), f"{rows}x{cols}: t={t} differs from t={n}"
        # the F64 closed form of the head at 17 tokens is minutes of CPU: its parity is test_head_parity's
        if not head:
            assert_parity(full, oracle.gemm_f64(h.q8, rows, cols, X), f"{rows}x{cols} t={n}")
    finally:
        h.close()


@pytest.mark.parametrize("rows,cols,ts", [(1888, 512, GATE_T), (16, 512, (2, 8, 16)), (64, 512, (2, 8, 16)), (512, 512, (2, 8, 16))])
def test_reference_gemm_gate(rt, oracle, rows, cols, ts):
    """The reference's own gemm gate on its own shapes (scripts/check.sh:132-149: 1888x512 at every
    token count of GATE_T, and 16, 64, 512 rows at 2, 8, 16 tokens): the reference-order kernel
    keeps gemm(t)[k] == gemv(x[k]) bit for bit and equals the oracle's F32 order; the fast kernels
    hold the parity bar against F64 at every t."""
    h = Handle(rt, rows, cols, seed=7 * rows + cols)
    try:
        X = np.random.default_rng(rows + 17).standard_normal((max(ts), cols), dtype=np.float32)
        one = np.concatenate([h.product(X[k], exact=True) for k in range(max(ts))])
        f64 = oracle.gemm_f64(h.q8, rows, cols, X)
        ref = oracle.gemm(h.q8, rows, cols, X)
        assert np.array_equal(one.view(np.uint32), ref.view(np.uint32)), "one token at a time against the oracle's F32 order"
        for t in ts:
            say(f"gate {rows}x{cols} t={t}")
            y = h.product(X[:t], exact=True)
            assert np.array_equal(y.view(np.uint32), one[:t].view(np.uint32)), f"reference order t={t}"
            assert_parity(h.product(X[:t]), f64[:t], f"fast t={t}")
    finally:
        h.close()
