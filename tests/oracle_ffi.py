"""The CPU oracle (oracle/liboracle.so) and the reference's compiled host model (oracle/_ref/libref.so),
bound with ctypes for the tests. Test infrastructure: the checker, never the thing checked.
"""
import ctypes as c
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libref.so")

_vp, _l = c.c_void_p, c.c_long


def _p(a):
    return c.c_void_p(a.ctypes.data)


def _build_if_missing():
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-C", ORACLE_DIR, "liboracle.so"], check=True, capture_output=True)


class Oracle:
    def __init__(self):
        _build_if_missing()
        self.lib = c.CDLL(ORACLE_SO)
        L = self.lib
        L.q8o_half.restype = c.c_float
        L.q8o_half.argtypes = [c.c_uint16]
        L.q8o_gemm.argtypes = [_vp, _l, _l, _vp, _l, _l, _vp]
        L.q8o_gemm_mt.argtypes = [_vp, _l, _l, _vp, _l, _l, _vp, c.c_int]
        L.q8o_gemm_f64.argtypes = [_vp, _l, _l, _vp, _l, _l, _vp]
        L.q8o_gemm_f64d.argtypes = [_vp, _l, _l, _vp, _l, _vp]
        L.q8o_rmsnorm_f64.argtypes = [_vp, _l, _l, _l, _vp, c.c_double, _vp]
        L.q8o_swiglu_f64.argtypes = [_vp, _vp, _l, _vp]
        L.q8o_repack_s.argtypes = [_vp, _l, _l, _vp]
        L.q8o_gate_a.argtypes = [_vp]
        L.q8o_gate21.argtypes = [_vp]
        L.q8o_gate21_inputs.argtypes = [_vp] * 6
        L.q8o_gate21_arrays.argtypes = [_vp, _vp]
        L.q8o_hash.restype = c.c_uint64
        L.q8o_hash.argtypes = [_vp, _l]
        L.q8o_row.argtypes = [_vp, _l, _l, _vp]
        L.q8o_next.restype = _l
        L.q8o_next.argtypes = [_vp, _l]

    def gemm(self, q8, rows, cols, x, threads=0):
        """Y [t rows] in the reference's F32 order; x [t cols] or [cols]."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
        t = x.shape[0]
        y = np.empty((t, rows), np.float32)
        if threads:
            self.lib.q8o_gemm_mt(_p(q8), rows, cols, _p(x), cols, t, _p(y), threads)
        else:
            self.lib.q8o_gemm(_p(q8), rows, cols, _p(x), cols, t, _p(y))
        return y

    def gemm_f64(self, q8, rows, cols, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
        t = x.shape[0]
        y = np.empty((t, rows), np.float64)
        self.lib.q8o_gemm_f64(_p(q8), rows, cols, _p(x), cols, t, _p(y))
        return y

    def gemm_f64d(self, q8, rows, cols, x):
        """F64 closed form with F64 x [t cols]."""
        x = np.ascontiguousarray(x, np.float64).reshape(-1, cols)
        y = np.empty((x.shape[0], rows), np.float64)
        self.lib.q8o_gemm_f64d(_p(q8), rows, cols, _p(x), x.shape[0], _p(y))
        return y

    def rmsnorm_f64(self, x, nw, eps):
        """The RMS norm of each row of x [t cols] in F64."""
        x = np.ascontiguousarray(x, np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        cols = x2.shape[1]
        out = np.empty(x2.shape, np.float64)
        self.lib.q8o_rmsnorm_f64(_p(x2), cols, x2.shape[0], cols, _p(np.ascontiguousarray(nw, np.float32)), float(eps), _p(out))
        return out

    def swiglu_f64(self, g, u):
        g = np.ascontiguousarray(g, np.float64)
        u = np.ascontiguousarray(u, np.float64)
        y = np.empty_like(g)
        self.lib.q8o_swiglu_f64(_p(g), _p(u), g.size, _p(y))
        return y

    def repack_s(self, q8, rows, cols):
        out = np.empty(rows * cols // 32 * 34, np.uint8)
        self.lib.q8o_repack_s(_p(q8), rows, cols, _p(out))
        return out

    def row(self, q8, cols, row):
        z = np.empty(cols, np.float32)
        self.lib.q8o_row(_p(q8), cols, row, _p(z))
        return z

    def next(self, a):
        a = np.ascontiguousarray(a, np.float32)
        return self.lib.q8o_next(_p(a), a.size)

    def half(self, h):
        return self.lib.q8o_half(int(h))

    def gate_a(self):
        out = (c.c_uint64 * 4)()
        self.lib.q8o_gate_a(out)
        return tuple(out)

    def gate21(self):
        out = (c.c_uint64 * 7)()
        self.lib.q8o_gate21(out)
        return tuple(out)

    def gate21_inputs(self):
        q = np.empty(512, np.int8)
        h = np.empty(131072, np.uint16)
        x8 = np.empty(512, np.float32)
        c8 = np.empty(512, np.float32)
        xf = np.empty(131072, np.float32)
        cf = np.empty(131072, np.float32)
        self.lib.q8o_gate21_inputs(_p(q), _p(h), _p(x8), _p(c8), _p(xf), _p(cf))
        return q, h, x8, c8, xf, cf

    def gate21_arrays(self):
        s8 = np.empty(512, np.float32)
        f16 = np.empty(131072, np.float32)
        self.lib.q8o_gate21_arrays(_p(s8), _p(f16))
        return s8, f16

    def hash(self, v):
        v = np.ascontiguousarray(v, np.float32)
        return self.lib.q8o_hash(_p(v), v.size)


class Reference:
    """The reference's own gemv.c / gemm.c / team.c, compiled from its sources into oracle/_ref."""

    def __init__(self, path=None):
        path = path or REF_SO
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = c.CDLL(path)
        L = self.lib
        L.ref_gemv.argtypes = [_vp, _l, _l, _vp, _vp]
        L.ref_gemm.argtypes = [_vp, _l, _l, _vp, _l, _vp]
        L.ref_repack_i.argtypes = [_vp, _l, _l, _vp]
        L.ref_gemv_i.argtypes = [_vp, _l, _l, _vp, _vp]
        L.ref_gemm_i.argtypes = [_vp, _l, _l, _vp, _l, _vp]
        L.ref_team_create.restype = _vp
        L.ref_team_create.argtypes = [c.c_int]
        L.ref_team_destroy.argtypes = [_vp]
        L.ref_team_gemv_i.argtypes = [_vp, _vp, _l, _l, _vp, _vp]
        L.ref_team_gemm_i.argtypes = [_vp, _vp, _l, _l, _vp, _l, _vp]
        L.rt_maxv.restype = c.c_float
        L.rt_maxv.argtypes = [_vp, _l]
        L.rt_index_of.restype = _l
        L.rt_index_of.argtypes = [_vp, _l, c.c_float]
        L.rt_q8_row.argtypes = [_vp, _l, _l, _vp]
        L.rt_sum.restype = c.c_float
        L.rt_sum.argtypes = [_vp, _l]
        for name in ("rt_s_div", "rt_s_add"):
            getattr(L, name).restype = c.c_float
            getattr(L, name).argtypes = [c.c_float, c.c_float]
        L.rt_s_rsqrt.restype = c.c_float
        L.rt_s_rsqrt.argtypes = [c.c_float]

    def gemm(self, q8, rows, cols, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
        t = x.shape[0]
        y = np.empty((t, rows), np.float32)
        self.lib.ref_gemm(_p(q8), rows, cols, _p(x), t, _p(y))
        return y

    def gemv(self, q8, rows, cols, x):
        y = np.empty(rows, np.float32)
        self.lib.ref_gemv(_p(q8), rows, cols, _p(np.ascontiguousarray(x, np.float32)), _p(y))
        return y

    def next(self, a):
        """rt_maxv then rt_index_of, as the generated code's Next runs them (a padded to whole
        16-lane blocks, as the runtime's arrays are, src/card/rt.h:5-8)."""
        n = a.size
        buf = np.zeros((n + 15) // 16 * 16 + 16, np.float32)
        buf[:n] = a
        m = self.lib.rt_maxv(_p(buf), n)
        return self.lib.rt_index_of(_p(buf), n, m)

    def row(self, q8, rows, cols, row):
        """rt_q8_row on the form I repack of GGUF rows."""
        fi = self.repack_i(q8, rows, cols)
        z = np.empty(cols + 16, np.float32)
        self.lib.rt_q8_row(_p(fi), cols, row, _p(z))
        return z[:cols]

    def rmsnorm_f32(self, x, nw, eps):
        """RMS of one row in the reference's F32 host arithmetic: x*x (one rounding, as the host
        loops' multiply), rt_sum over it, rt_s_div by the length, rt_s_add of eps, rt_s_rsqrt,
        then nw * (x * s) (src/apl/qwen35.apl:49; src/card/rt.c:106-135)."""
        x = np.ascontiguousarray(x, np.float32)
        n = x.size
        sq = np.zeros((n + 15) // 16 * 16, np.float32)
        sq[:n] = x * x
        ss = self.lib.rt_sum(_p(sq), n)
        s = self.lib.rt_s_rsqrt(self.lib.rt_s_add(np.float32(eps), self.lib.rt_s_div(ss, np.float32(n))))
        return np.asarray(nw, np.float32) * (x * np.float32(s))

    def repack_i(self, q8, rows, cols):
        out = np.empty(rows * cols // 32 * 34, np.uint8)
        self.lib.ref_repack_i(_p(q8), rows, cols, _p(out))
        return out


def reference_or_none():
    try:
        return Reference()
    except (FileNotFoundError, OSError):
        return None
