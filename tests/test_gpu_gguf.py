"""The GGUF load path on the GPU: rt_gguf_upload puts every Q8_0 tensor of a file in HBM once per
distinct offset (tied tensors share one handle, src/card/engine.c:307-310), through pinned staging
in chunks of whole 16-row groups.

Pinned by the bytes: each handle's device bytes equal the oracle's form S of the tensor's rows as
they lie in the file, and a product on it equals the product on the same rows uploaded from host
memory; every row read gives the oracle's d * q bit for bit."""
import ctypes as c
import os

import numpy as np
import pytest

import gguf_file as gf
import synth

pytestmark = pytest.mark.gpu

SHAPES = {"token_embd.weight": (64, 256), "blk.0.ffn_gate.weight": (96, 256), "blk.0.ffn_down.weight": (256, 96),
          "blk.0.attn_qkv.weight": (48, 1024)}


def _device_bytes(rt, w, nbytes):
    out = np.empty(nbytes, np.uint8)
    rt.lib.rt_dev_download(rt.R, out.ctypes.data_as(c.c_void_p), c.c_void_p(w), nbytes)
    return out


@pytest.mark.parametrize("chunk", [None, 4352])
def test_gguf_upload_bytes_rows_products(rt, q8rt, oracle, tmp_path, chunk):
    """Every Q8_0 tensor: its HBM bytes are the oracle's form S of the file's rows, rows read back
    bit for bit, and a product equals the host-memory upload's. chunk = 4352 B (one 16-row group
    of 256 columns) makes every matrix cross several chunks, the last one partial."""
    keys, tensors, q8 = gf.model(23, SHAPES, alignment=64)
    path = tmp_path / "model.gguf"
    gf.write(path, keys, tensors, alignment=64)
    old = rt.set_upload_chunk(chunk) if chunk else None
    try:
        g = q8rt.GGUF(path)
        g.upload(rt)
    finally:
        if chunk:
            rt.set_upload_chunk(old)
    try:
        assert g.h.q8_count == len(SHAPES)
        assert g.h.q8_bytes == sum(r * k // 32 * 34 for r, k in SHAPES.values())
        rng = np.random.default_rng(3)
        for name, (rows, cols) in SHAPES.items():
            t = g.tensor(name)
            assert t["w"], name
            assert np.array_equal(_device_bytes(rt, t["w"], t["bytes"]), oracle.repack_s(q8[name], rows, cols)), name
            for r in (0, 15, 16, rows - 1):
                z = np.empty(cols, np.float32)
                rt.lib.rt_q8_row(c.c_void_p(t["w"]), cols, r, z.ctypes.data_as(c.c_void_p))
                assert np.array_equal(z.view(np.uint32), oracle.row(q8[name], cols, r).view(np.uint32)), (name, r)
            x = rng.standard_normal(cols).astype(np.float32)
            y_file, y_host = np.empty(rows, np.float32), np.empty(rows, np.float32)
            h = rt.upload(q8[name], rows, cols)
            try:
                rt.gemv(t["w"], rows, cols, x, y_file)
                rt.gemv(h, rows, cols, x, y_host)
            finally:
                rt.lib.rt_q8_free(rt.R, c.c_void_p(h))
            assert np.array_equal(y_file.view(np.uint32), y_host.view(np.uint32)), name
        # tied by offset: one handle for both names
        assert g.tensor("output.weight")["w"] == g.tensor("token_embd.weight")["w"]
        assert g.tensor("output_norm.weight")["w"] is None
    finally:
        g.release()
    assert all(t["w"] is None for t in g.tensors()) and g.h.q8_count == 0
    g.close()


def test_gguf_upload_refuses_a_bad_matrix_and_leaves_nothing(rt, q8rt, tmp_path):
    """A Q8_0 tensor the products cannot take (40 rows) after good ones: the upload fails naming
    it, and the handles already made are freed."""
    rng = np.random.default_rng(4)
    good = synth.q8_rows(rng, 32, 256)
    bad = synth.q8_rows(rng, 40, 256)
    tensors = [{"name": "a.weight", "dims": [256, 32], "type": gf.Q8_0, "data": good.tobytes()},
               {"name": "b.weight", "dims": [256, 40], "type": gf.Q8_0, "data": bad.tobytes()}]
    path = tmp_path / "bad.gguf"
    gf.write(path, [], tensors)
    with q8rt.GGUF(path) as g:
        with pytest.raises(RuntimeError, match="tensor b.weight: 40 rows x 256 columns is not a matrix"):
            g.upload(rt)
        assert all(t["w"] is None for t in g.tensors()) and g.h.q8_count == 0 and g.h.q8_bytes == 0


def test_gguf_upload_fd_reads_at_offset(rt, q8rt, oracle, tmp_path):
    """rt_q8_upload_fd on its own: a matrix at an odd offset of a file (not a GGUF), several chunks."""
    rows, cols = 80, 512
    q8, _ = synth.case(31, rows, cols, 1)
    path = tmp_path / "raw.bin"
    path.write_bytes(b"\x07" * 1001 + q8.tobytes() + b"\x09" * 17)
    fd = os.open(path, os.O_RDONLY)
    old = rt.set_upload_chunk(3 * 16 * cols // 32 * 34)
    try:
        w = rt.lib.rt_q8_upload_fd(rt.R, fd, 1001, rows, cols)
    finally:
        os.close(fd)
        rt.set_upload_chunk(old)
    assert w
    try:
        assert np.array_equal(_device_bytes(rt, w, q8.size), oracle.repack_s(q8, rows, cols))
    finally:
        rt.lib.rt_q8_free(rt.R, c.c_void_p(w))
