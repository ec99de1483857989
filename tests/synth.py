"""Seeded synthetic Q8_0 weights and activations on the host, in the configurations' distributions:
q uniform integers in [-127, 127]; d = binary16(|N(0, 0.02)| / 127), or binary16(lognormal(ln 0.002, 1.0))
for the heavy-tailed verify configuration; x ~ N(0, 1) in F32. numpy's PCG64 stream, drawn in the
order q, d, x. The GPU benchmark draws the same distributions on the device (rt_q8_fill_dev).
"""
import numpy as np


def q8_rows(rng, rows, cols, dist="normal"):
    """GGUF Q8_0 rows: per 32 columns a binary16 scale then 32 int8; flat uint8."""
    nb = cols // 32
    q = rng.integers(-127, 128, size=(rows, nb, 32), dtype=np.int8)
    if dist == "normal":
        d = (np.abs(rng.normal(0.0, 0.02, size=(rows, nb))) / 127.0).astype(np.float16)
    elif dist == "lognormal":
        d = rng.lognormal(np.log(0.002), 1.0, size=(rows, nb)).astype(np.float16)
    else:
        raise ValueError(dist)
    blk = np.empty((rows, nb, 34), np.uint8)
    blk[:, :, :2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = q.view(np.uint8)
    return blk.reshape(-1)


def x_f32(rng, t, cols):
    return rng.standard_normal(size=(t, cols), dtype=np.float32)


def case(seed, rows, cols, t, dist="normal"):
    rng = np.random.default_rng(seed)
    q8 = q8_rows(rng, rows, cols, dist)
    x = x_f32(rng, t, cols)
    return q8, x


def split(q8, rows, cols):
    """(q int8 [rows cols], d float16 [rows cols/32]) views of GGUF rows."""
    nb = cols // 32
    blk = q8.reshape(rows, nb, 34)
    d = np.ascontiguousarray(blk[:, :, :2]).view(np.float16).reshape(rows, nb)
    q = np.ascontiguousarray(blk[:, :, 2:]).view(np.int8).reshape(rows, cols)
    return q, d


def join(q, d):
    """GGUF rows from q int8 [rows cols] and d float16 [rows cols/32]."""
    rows, cols = q.shape
    nb = cols // 32
    blk = np.empty((rows, nb, 34), np.uint8)
    blk[:, :, :2] = np.ascontiguousarray(d, np.float16).view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = np.ascontiguousarray(q, np.int8).view(np.uint8).reshape(rows, nb, 32)
    return blk.reshape(-1)
