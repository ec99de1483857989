"""Python view of libq8rt.so, the MI355X Q8_0 weight products (include/q8_rt.h).

The product is the C-ABI: this module binds it with ctypes for the tests and the benchmark,
names every symbol the header declares, and wraps a `struct rt` in `Runtime`. It computes
nothing itself: every product runs in the HIP kernels of libq8rt.so, and a missing library
is an error (RuntimeError), never a fallback.

Reference interface mirrored: src/card/rt.h:19-26 (struct rt), 38-39 (rt_init), 61-72
(rt_gemv, rt_gemv_q, rt_gemv_open, rt_gemv_go, rt_gemm, rt_gemm_q); src/card/gemv.h:50-57
(gemv_i_bytes, gemv_i_repack); src/host/gguf_reader.h:17-58 (the GGUF header reader, as
rt_gguf_*, include/q8_gguf.h) and src/card/engine.c:287-316 (the load loop, rt_gguf_upload).
"""
import glob
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq8rt.so")
HEADERS = sorted(glob.glob(os.path.join(os.path.dirname(HERE), "include", "*.h")))

_c = ctypes
_vp, _long, _int, _f32p, _u64 = _c.c_void_p, _c.c_long, _c.c_int, _c.c_void_p, _c.c_uint64


class Rt(_c.Structure):
    """struct rt, field for field (src/card/rt.h:19-26)."""

    _fields_ = [("team", _vp), ("frame", _c.c_char_p), ("chain", _vp), ("gemm_chain", _vp), ("threads", _int), ("last", _int)]


# name -> (restype, argtypes)
_SIGS = {
    "rt_init": (_int, [_vp, _int]),
    "rt_fini": (None, [_vp]),
    "rt_gemv": (None, [_vp, _vp, _long, _long, _vp, _vp]),
    "rt_gemv_q": (None, [_vp, _vp, _long, _long, _vp, _vp]),
    "rt_gemv_open": (None, [_vp]),
    "rt_gemv_go": (None, [_vp]),
    "rt_gemm": (None, [_vp, _vp, _long, _long, _vp, _long, _vp]),
    "rt_gemm_q": (None, [_vp, _vp, _long, _long, _vp, _long, _vp]),
    "gemv_i_bytes": (_long, [_long, _long]),
    "gemv_i_repack": (None, [_vp, _long, _long, _vp]),
    "rt_q8_upload": (_vp, [_vp, _vp, _long, _long]),
    "rt_q8_upload_packed": (_vp, [_vp, _vp, _long, _long]),
    "rt_q8_free": (None, [_vp, _vp]),
    "rt_gemv_dev": (None, [_vp, _vp, _long, _long, _vp, _vp]),
    "rt_gemm_dev": (None, [_vp, _vp, _long, _long, _vp, _long, _long, _vp]),
    "rt_gemm_dev_noalloc": (None, [_vp, _vp, _long, _long, _vp, _long, _long, _vp]),
    "rt_gemv_swiglu_dev": (None, [_vp, _vp, _vp, _long, _long, _vp, _long, _long, _vp]),
    "rt_gemv_round_dev": (None, [_vp, _int, _vp, _vp, _long, _vp, _long, _long, _vp]),
    "rt_dev_alloc": (_vp, [_vp, _long]),
    "rt_dev_free": (None, [_vp, _vp]),
    "rt_dev_upload": (None, [_vp, _vp, _vp, _long]),
    "rt_dev_download": (None, [_vp, _vp, _vp, _long]),
    "rt_dev_sync": (None, [_vp]),
    "rt_q8_fill_dev": (None, [_vp, _vp, _long, _long, _u64, _int, _c.c_float, _c.c_float]),
    "rt_q8_repack_dev": (None, [_vp, _vp, _long, _long, _vp]),
    "rt_f32_fill_dev": (None, [_vp, _vp, _long, _u64]),
    "rt_dev_copy": (None, [_vp, _vp, _vp, _long]),
    "rt_q8_read_dev": (None, [_vp, _vp, _vp, _long, _long, _vp, _long, _long, _vp]),
    "rt_q8_row": (None, [_vp, _long, _long, _vp]),
    "rt_q8_rows_dev": (None, [_vp, _vp, _long, _vp, _long, _vp]),
    "rt_argmax_dev": (None, [_vp, _vp, _long, _vp]),
    "rt_prims_dev": (None, [_vp, _vp, _vp, _vp, _vp, _long, _vp, _vp, _vp, _vp, _long]),
    "rt_set_exact": (_int, [_vp, _int]),
    "rt_set_epi_apart": (_int, [_vp, _int]),
    "rt_set_x_direct": (_int, [_vp, _int]),
    "rt_set_upload_chunk": (_long, [_vp, _long]),
    "rt_gemm_force": (None, [_vp, _int, _int]),
    "rt_timer_start": (None, [_vp]),
    "rt_timer_stop": (_c.c_float, [_vp]),
    "rt_device_info": (None, [_vp, _c.c_char_p, _long, _c.POINTER(_int)]),
    "rt_graph_begin": (None, [_vp]),
    "rt_graph_end": (_vp, [_vp]),
    "rt_graph_launch": (None, [_vp, _vp]),
    "rt_graph_free": (None, [_vp, _vp]),
    "rt_ktime": (None, [_vp, _int]),
    "rt_host_timing": (None, [_vp, _int]),
    "rt_host_timing_read": (_long, [_vp, _vp]),
    "rt_ktime_read": (_long, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _long]),
    "rt_q8_upload_fd": (_vp, [_vp, _int, _u64, _long, _long]),
    "rt_rmsnorm_dev": (None, [_vp, _vp, _long, _long, _long, _vp, _c.c_float, _vp]),
    "rt_gemm_norm_dev": (None, [_vp, _vp, _long, _long, _vp, _long, _long, _vp, _c.c_float, _vp]),
    "rt_gemv_swiglu_norm_dev": (None, [_vp, _vp, _vp, _long, _long, _vp, _long, _long, _vp, _c.c_float, _vp]),
    "rt_gemv_round_norm_dev": (None, [_vp, _int, _vp, _vp, _long, _vp, _long, _long, _vp, _c.c_float, _vp]),
    "rt_gemm_residual_dev": (None, [_vp, _vp, _long, _long, _vp, _long, _long, _vp, _vp]),
    "rt_gguf_read": (_int, [_vp, _c.c_char_p, _c.c_char_p, _c.c_size_t]),
    "rt_gguf_free": (None, [_vp]),
    "rt_gguf_key": (_vp, [_vp, _c.c_char_p]),
    "rt_gguf_tensor": (_vp, [_vp, _c.c_char_p]),
    "rt_gguf_tensor_at": (_vp, [_vp, _u64]),
    "rt_gguf_key_u64": (_u64, [_vp, _c.c_char_p, _u64]),
    "rt_gguf_value_type_name": (_c.c_char_p, [_c.c_uint32]),
    "rt_gguf_tensor_type_name": (_c.c_char_p, [_c.c_uint32]),
    "rt_gguf_upload": (_int, [_vp, _vp, _c.c_char_p, _c.c_char_p, _c.c_size_t]),
    "rt_gguf_release": (None, [_vp, _vp]),
}


class GgufKey(_c.Structure):
    """struct rt_gguf_key (include/q8_gguf.h; gguf_reader.h:17-23)."""

    _fields_ = [("name", _c.c_char * 96), ("type", _c.c_uint32), ("elem_type", _c.c_uint32), ("n", _u64), ("text", _c.c_char * 128)]


class GgufTensor(_c.Structure):
    """struct rt_gguf_tensor (include/q8_gguf.h; gguf_reader.h:25-32, plus the HBM handle)."""

    _fields_ = [("name", _c.c_char * 96), ("n_dims", _c.c_uint32), ("dim", _u64 * 4), ("type", _c.c_uint32), ("offset", _u64), ("bytes", _u64),
                ("w", _vp)]


class GgufHeader(_c.Structure):
    """struct rt_gguf (include/q8_gguf.h; gguf_reader.h:34-43, plus the upload's totals)."""

    _fields_ = [("version", _c.c_uint32), ("file_size", _u64), ("header_end", _u64), ("data_start", _u64), ("data_bytes", _u64), ("need", _u64),
                ("n_keys", _u64), ("n_tensors", _u64), ("keys", _c.POINTER(GgufKey)), ("tensors", _c.POINTER(GgufTensor)), ("q8_bytes", _u64),
                ("q8_count", _int)]

KINDS = {0: "gemv", 1: "gemv_pair", 2: "gemm", 3: "gemm_pair", 4: "exact", 5: "round"}


def header_symbols(paths=None):
    """Every function name the headers under include/ declare."""
    names = set()
    for path in paths or HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
        names |= set(re.findall(r"^[A-Za-z_][\w \*]*?\b(\w+)\s*\(", text, flags=re.M))
    return sorted(names - {"defined"})


_lib = None


def load():
    """The library, its signatures set. RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run `make -C {HERE}` or __graft_entry__.build()")
    lib = _c.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def ptr(a):
    """The address of a numpy array's data (or an int address) as a c_void_p."""
    if isinstance(a, int):
        return _c.c_void_p(a)
    if a is None:
        return _c.c_void_p(0)
    return _c.c_void_p(a.ctypes.data)


class Runtime:
    """One `struct rt` with rt_init done; the GPU context lives until close()."""

    def __init__(self, threads=1):
        self.lib = load()
        self.rt = Rt()
        if self.lib.rt_init(_c.byref(self.rt), threads) != 0:
            raise RuntimeError("rt_init failed: no GPU visible, or no memory for the runtime")
        self.R = _c.byref(self.rt)

    def close(self):
        if self.rt.chain:
            self.lib.rt_fini(self.R)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- the reference's entry points, host arrays (numpy float32, C-contiguous)
    def upload(self, q8, rows, cols):
        h = self.lib.rt_q8_upload(self.R, ptr(q8), rows, cols)
        if not h:
            raise MemoryError("rt_q8_upload: HBM is full")
        return h

    def gemv(self, w, rows, cols, x, y):
        self.lib.rt_gemv(self.R, _c.c_void_p(w), rows, cols, ptr(x), ptr(y))

    def gemm(self, w, rows, cols, x, t, y):
        self.lib.rt_gemm(self.R, _c.c_void_p(w), rows, cols, ptr(x), t, ptr(y))

    def gemv_q(self, w, rows, cols, x, y):
        self.lib.rt_gemv_q(self.R, _c.c_void_p(w), rows, cols, ptr(x), ptr(y))

    def gemm_q(self, w, rows, cols, x, t, y):
        self.lib.rt_gemm_q(self.R, _c.c_void_p(w), rows, cols, ptr(x), t, ptr(y))

    def gemv_open(self):
        self.lib.rt_gemv_open(self.R)

    def gemv_go(self):
        self.lib.rt_gemv_go(self.R)

    def set_exact(self, on):
        return self.lib.rt_set_exact(self.R, 1 if on else 0)

    def set_epi_apart(self, on):
        return self.lib.rt_set_epi_apart(self.R, 1 if on else 0)

    def set_x_direct(self, on):
        return self.lib.rt_set_x_direct(self.R, 1 if on else 0)

    def set_upload_chunk(self, nbytes):
        return self.lib.rt_set_upload_chunk(self.R, int(nbytes))

    def gemm_force(self, streaming=False, ks=0):
        """The matrix-core product's kernel and K split for the following products (a test hook;
        gemm_force() restores the planner's)."""
        self.lib.rt_gemm_force(self.R, 1 if streaming else 0, int(ks))

    # ---- device memory
    def alloc(self, nbytes):
        p = self.lib.rt_dev_alloc(self.R, int(nbytes))
        if not p:
            raise MemoryError(f"rt_dev_alloc({nbytes})")
        return p

    def free(self, p):
        self.lib.rt_dev_free(self.R, _c.c_void_p(p))

    def to_dev(self, dst, a):
        self.lib.rt_dev_upload(self.R, _c.c_void_p(dst), ptr(a), a.nbytes)

    def from_dev(self, a, src):
        self.lib.rt_dev_download(self.R, ptr(a), _c.c_void_p(src), a.nbytes)

    def sync(self):
        self.lib.rt_dev_sync(self.R)

    def device_info(self):
        name = _c.create_string_buffer(256)
        cus = _int(0)
        self.lib.rt_device_info(self.R, name, 256, _c.byref(cus))
        return name.value.decode(), cus.value


class GGUF:
    """A GGUF file's header and tensor table (rt_gguf_read) and, after upload(runtime), the HBM
    handles of its Q8_0 tensors (rt_gguf_upload: one per distinct file offset, so tensors tied by
    offset share one). A bad file raises ValueError with the library's "path: reason"."""

    def __init__(self, path):
        self.lib = load()
        self.path = os.fsencode(path)
        self.h = GgufHeader()
        self.runtime = None
        err = _c.create_string_buffer(512)
        if self.lib.rt_gguf_read(_c.byref(self.h), self.path, err, 512) != 0:
            raise ValueError(err.value.decode())

    @staticmethod
    def _key(k):
        return {"name": k.name.decode(), "type": k.type, "elem_type": k.elem_type, "n": k.n, "text": k.text.decode()}

    @staticmethod
    def _tensor(t):
        return {"name": t.name.decode(), "n_dims": t.n_dims, "dim": list(t.dim), "type": t.type, "offset": t.offset, "bytes": t.bytes,
                "w": t.w}

    def keys(self):
        return [self._key(self.h.keys[i]) for i in range(self.h.n_keys)]

    def tensors(self):
        return [self._tensor(self.h.tensors[i]) for i in range(self.h.n_tensors)]

    def tensor(self, name):
        p = self.lib.rt_gguf_tensor(_c.byref(self.h), name.encode())
        return self._tensor(GgufTensor.from_address(p)) if p else None

    def tensor_at(self, offset):
        p = self.lib.rt_gguf_tensor_at(_c.byref(self.h), offset)
        return self._tensor(GgufTensor.from_address(p)) if p else None

    def key(self, name):
        p = self.lib.rt_gguf_key(_c.byref(self.h), name.encode())
        return self._key(GgufKey.from_address(p)) if p else None

    def key_u64(self, name, fallback=0):
        return self.lib.rt_gguf_key_u64(_c.byref(self.h), name.encode(), fallback)

    def upload(self, runtime):
        """Every Q8_0 tensor to HBM; RuntimeError with the reason (nothing left uploaded) if not."""
        err = _c.create_string_buffer(512)
        if self.lib.rt_gguf_upload(runtime.R, _c.byref(self.h), self.path, err, 512) != 0:
            raise RuntimeError(err.value.decode())
        self.runtime = runtime

    def release(self):
        if self.runtime is not None:
            self.lib.rt_gguf_release(self.runtime.R, _c.byref(self.h))
            self.runtime = None

    def close(self):
        self.release()
        self.lib.rt_gguf_free(_c.byref(self.h))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
