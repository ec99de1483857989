"""The GGUF header reader (rt_gguf_read, include/q8_gguf.h) on synthetic GGUF v3 files.

Pinned three ways: against the reference's own reader (src/host/gguf_reader.c, built from its source
into oracle/_ref/libgguf.so) field for field and error for error; against the writer's own byte
accounting (where the header ends, where the data starts, every tensor's offset and size), which
needs no reference; and on the error paths the reference defines (gguf_reader.c:60-160). No GPU."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import gguf_file as gf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_GGUF = os.path.join(ROOT, "oracle", "_ref", "libgguf.so")


class RefKey(C.Structure):
    _fields_ = [("name", C.c_char * 96), ("type", C.c_uint32), ("elem_type", C.c_uint32), ("n", C.c_uint64), ("text", C.c_char * 128)]


class RefTensor(C.Structure):
    _fields_ = [("name", C.c_char * 96), ("n_dims", C.c_uint32), ("dim", C.c_uint64 * 4), ("type", C.c_uint32), ("offset", C.c_uint64),
                ("bytes", C.c_uint64)]


class RefGguf(C.Structure):
    """struct gguf of src/host/gguf_reader.h:34-43."""

    _fields_ = [("version", C.c_uint32), ("file_size", C.c_uint64), ("header_end", C.c_uint64), ("data_start", C.c_uint64),
                ("data_bytes", C.c_uint64), ("need", C.c_uint64), ("n_keys", C.c_uint64), ("n_tensors", C.c_uint64),
                ("keys", C.POINTER(RefKey)), ("tensors", C.POINTER(RefTensor))]


@pytest.fixture(scope="module")
def ref_gguf():
    if not os.path.exists(REF_GGUF):
        pytest.skip("oracle/_ref/libgguf.so is not built (the reference's sources are not here)")
    lib = C.CDLL(REF_GGUF)
    lib.gguf_load.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_size_t]
    lib.gguf_load.restype = C.c_int
    lib.gguf_free.argtypes = [C.c_void_p]
    lib.gguf_key_u64.argtypes = [C.c_void_p, C.c_char_p, C.c_uint64]
    lib.gguf_key_u64.restype = C.c_uint64
    lib.gguf_tensor_type_name.argtypes = [C.c_uint32]
    lib.gguf_tensor_type_name.restype = C.c_char_p
    lib.gguf_value_type_name.argtypes = [C.c_uint32]
    lib.gguf_value_type_name.restype = C.c_char_p
    return lib


def ref_read(lib, path):
    g = RefGguf()
    err = C.create_string_buffer(512)
    rc = lib.gguf_load(C.byref(g), os.fsencode(path), err, 512)
    if rc != 0:
        return None, err.value.decode()
    head = {f: getattr(g, f) for f in ("version", "file_size", "header_end", "data_start", "data_bytes", "need", "n_keys", "n_tensors")}
    keys = [{"name": g.keys[i].name.decode(), "type": g.keys[i].type, "elem_type": g.keys[i].elem_type, "n": g.keys[i].n,
             "text": g.keys[i].text.decode()} for i in range(g.n_keys)]
    tensors = [{"name": t.name.decode(), "n_dims": t.n_dims, "dim": list(t.dim), "type": t.type, "offset": t.offset, "bytes": t.bytes}
               for t in (g.tensors[i] for i in range(g.n_tensors))]
    u64 = {k["name"]: lib.gguf_key_u64(C.byref(g), k["name"].encode(), 77) for k in keys}
    lib.gguf_free(C.byref(g))
    return (head, keys, tensors, u64), None


def our_read(q8rt, path):
    try:
        g = q8rt.GGUF(path)
    except ValueError as e:
        return None, str(e)
    head = {f: getattr(g.h, f) for f in ("version", "file_size", "header_end", "data_start", "data_bytes", "need", "n_keys", "n_tensors")}
    tensors = [{k: v for k, v in t.items() if k != "w"} for t in g.tensors()]
    keys = g.keys()
    u64 = {k["name"]: g.key_u64(k["name"], 77) for k in keys}
    g.close()
    return (head, keys, tensors, u64), None


# every scalar type at its extremes, strings short, empty and longer than the 127 kept bytes, and
# arrays: numeric of up to 16 elements (printed), of 17 (skipped), of strings (skipped), empty
KEYS_ALL = [
    ("general.architecture", gf.STR, "qwen35"),
    ("general.name", gf.STR, "n" * 300),
    ("general.empty", gf.STR, ""),
    ("k.u8", gf.U8, 255), ("k.i8", gf.I8, -128), ("k.u16", gf.U16, 65535), ("k.i16", gf.I16, -32768),
    ("k.u32", gf.U32, 4294967295), ("k.i32", gf.I32, -2147483648), ("k.f32", gf.F32, 1e-6), ("k.f32pi", gf.F32, 3.14159274),
    ("k.f32neg", gf.F32, -0.0), ("k.bool0", gf.BOOL, 0), ("k.bool1", gf.BOOL, 1), ("k.u64", gf.U64, 2**64 - 1),
    ("k.i64", gf.I64, -2**63), ("k.f64", gf.F64, 2.718281828459045), ("k.f64tiny", gf.F64, 5e-324),
    ("a.u32", gf.ARR, (gf.U32, [1, 2, 3, 4])),
    ("a.f32x16", gf.ARR, (gf.F32, [i / 3 for i in range(16)])),
    ("a.f64x16", gf.ARR, (gf.F64, [i / 7 for i in range(16)])),
    ("a.i64x17", gf.ARR, (gf.I64, list(range(17)))),
    ("a.str", gf.ARR, (gf.STR, ["a", "bb", "c" * 40])),
    ("a.bool", gf.ARR, (gf.BOOL, [1, 0, 1])),
    ("a.empty", gf.ARR, (gf.I8, [])),
    ("qwen35.embedding_length", gf.U32, 256),
]

TENSORS_ALL = [
    {"name": "token_embd.weight", "dims": [256, 64], "type": gf.Q8_0},
    {"name": "output_norm.weight", "dims": [256], "type": gf.F32_T},
    {"name": "blk.0.odd.weight", "dims": [100], "type": gf.F16_T},
    {"name": "blk.0.q4.weight", "dims": [64, 3], "type": gf.Q4_0},
    {"name": "blk.0.cube.weight", "dims": [64, 4, 8], "type": gf.Q8_0},
    {"name": "blk.0.four.weight", "dims": [2, 3, 4, 5], "type": gf.F32_T},
    {"name": "blk.0.k.weight", "dims": [256, 2], "type": 12},
    {"name": "blk.0.bf.weight", "dims": [7], "type": 30},
    {"name": "output.weight", "dims": [256, 64], "type": gf.Q8_0, "tie": "token_embd.weight"},
]


@pytest.mark.parametrize("alignment", [32, 64, 1, 4096])
def test_header_matches_reference(q8rt, ref_gguf, tmp_path, alignment):
    keys = list(KEYS_ALL) + ([("general.alignment", gf.U32, alignment)] if alignment != 32 else [])
    path = tmp_path / "m.gguf"
    gf.write(path, keys, TENSORS_ALL, alignment=alignment)
    ours, e1 = our_read(q8rt, path)
    ref, e2 = ref_read(ref_gguf, path)
    assert e1 is None and e2 is None, (e1, e2)
    assert ours[0] == ref[0]
    assert ours[1] == ref[1]
    assert ours[2] == ref[2]
    assert ours[3] == ref[3]


def test_header_known_answer(q8rt, tmp_path):
    """Offsets and sizes against the writer's own accounting (no reference needed)."""
    for alignment in (32, 64, 1):
        keys = list(KEYS_ALL) + ([("general.alignment", gf.U32, alignment)] if alignment != 32 else [])
        path = tmp_path / f"m{alignment}.gguf"
        info = gf.write(path, keys, TENSORS_ALL, alignment=alignment)
        with q8rt.GGUF(path) as g:
            h = g.h
            assert (h.version, h.n_keys, h.n_tensors) == (3, len(keys), len(TENSORS_ALL))
            assert h.header_end == info["header_end"] and h.data_start == info["data_start"]
            assert h.file_size == info["size"] == os.path.getsize(path)
            ends = []
            for spec, t in zip(TENSORS_ALL, g.tensors()):
                assert t["name"] == spec["name"] and t["dim"][:t["n_dims"]] == spec["dims"] and t["type"] == spec["type"]
                assert t["offset"] == info["offsets"][spec["name"]]
                assert t["bytes"] == gf.tensor_bytes(spec["dims"], spec["type"])
                ends.append(t["offset"] + t["bytes"])
            assert h.need == max(ends) == h.file_size
            assert h.data_bytes == sum(t["bytes"] for t in g.tensors())
            # tied by offset: the lookups by offset and by name agree
            emb, out = g.tensor("token_embd.weight"), g.tensor("output.weight")
            assert emb["offset"] == out["offset"] and g.tensor_at(emb["offset"])["name"] == "token_embd.weight"
            assert g.key("general.name")["text"] == "n" * 127 and g.key("general.name")["n"] == 300
            assert g.key("a.u32")["text"] == "1 2 3 4" and g.key("a.i64x17")["text"] == "" and g.key("a.i64x17")["n"] == 17
            assert g.key("k.bool1")["text"] == "true" and g.key("k.i8")["text"] == "-128"
            assert g.key_u64("qwen35.embedding_length", 0) == 256 and g.key_u64("absent", 9) == 9
            assert g.tensor("absent") is None and g.key("absent") is None


def test_type_names_match_reference(q8rt, ref_gguf):
    lib = q8rt.load()
    for t in range(0, 48):
        assert lib.rt_gguf_tensor_type_name(t) == ref_gguf.gguf_tensor_type_name(t), t
    for t in range(0, 16):
        assert lib.rt_gguf_value_type_name(t) == ref_gguf.gguf_value_type_name(t), t


def _bad_files(tmp_path):
    """(name, path) of malformed files; every one the reference also refuses."""
    out = []
    blob, info = gf.build(KEYS_ALL, TENSORS_ALL)

    def put(name, data):
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        out.append((name, p))

    put("magic", b"GGUX" + blob[4:])
    for cut in (2, 10, 20, 30, info["keys_end"] - 3, info["keys_end"] + 5, info["header_end"] - 5):
        put(f"cut{cut}", blob[:cut])
    put("value_type", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gf.gstr("k.bad") + struct.pack("<I", 13) + bytes(8))
    put("array_of_arrays", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gf.gstr("a.a") + struct.pack("<IIQ", gf.ARR, gf.ARR, 1))
    put("array_bad_elem", b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gf.gstr("a.b") + struct.pack("<IIQ", gf.ARR, 14, 40))
    five = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + gf.gstr("t") + struct.pack("<I", 5) + struct.pack("<5Q", 1, 1, 1, 1, 1) + struct.pack("<IQ", 0, 0)
    put("five_dims", five)
    for ty in (4, 31, 43, 1000):
        put(f"ggml_type{ty}", b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + gf.gstr("t") + struct.pack("<IQ", 1, 32) + struct.pack("<IQ", ty, 0))
    out.append(("missing", tmp_path / "no_such_file.gguf"))
    out.append(("directory", tmp_path))
    return out


def test_errors_match_reference(q8rt, ref_gguf, tmp_path):
    """Every malformed file the reference's reader refuses, this one refuses too (the texts differ:
    these name the byte where the header went wrong)."""
    for name, path in _bad_files(tmp_path):
        ours, e1 = our_read(q8rt, path)
        ref, e2 = ref_read(ref_gguf, path)
        assert ours is None and ref is None, (name, e1, e2)


def test_errors_known(q8rt, tmp_path):
    """The reasons, without the reference: each bad file names what is wrong, and where."""
    want = {"magic": 'not a GGUF file: it starts with 47 47 55 58, not "GGUF"', "five_dims": "a tensor has more than 4 dimensions (at byte",
            "value_type": "a key has a value type GGUF does not define (at byte",
            "array_of_arrays": "an array has an element type GGUF does not define (at byte",
            "array_bad_elem": "an array has an element type GGUF does not define (at byte", "missing": "No such file or directory",
            "directory": "Is a directory"}
    for name, path in _bad_files(tmp_path):
        _, e = our_read(q8rt, path)
        assert e.startswith(str(path) + ": "), e
        if name in want:
            assert want[name] in e, (name, e)
        elif name.startswith("cut"):
            assert "the header ends" in e and f"of {path.stat().st_size})" in e, (name, e)
        elif name.startswith("ggml_type"):
            assert "a tensor has a ggml type id this reader does not know (at byte" in e, (name, e)
    # the byte named is where the header went wrong: a cut at 10 bytes fails reading the tensor
    # count at byte 8, a value type 13 fails after the key's name and type
    cut10 = dict(_bad_files(tmp_path))["cut10"]
    assert our_read(q8rt, cut10)[1].endswith("(at byte 8 of 10)")
    vt = dict(_bad_files(tmp_path))["value_type"]
    assert our_read(q8rt, vt)[1].endswith(f"(at byte {24 + 8 + 5 + 4} of {vt.stat().st_size})")


def test_counts_beyond_the_file_refused_before_allocating(q8rt, tmp_path):
    """A header whose key or tensor count the rest of the file cannot hold (a corrupt count of 2^60)
    is refused with that reason, without allocating tables for it."""
    import struct as st
    for nt, nk in ((1 << 60, 0), (0, 1 << 60), (2, 0)):
        path = tmp_path / f"counts{nt}_{nk}.gguf"
        path.write_bytes(b"GGUF" + st.pack("<IQQ", 3, nt, nk) + bytes(20))
        _, e = our_read(q8rt, path)
        assert "counts larger than the file holds" in e, e


def test_zero_alignment_is_an_error(q8rt, tmp_path):
    """An alignment of 0 (the reference divides by it) is refused."""
    path = tmp_path / "a0.gguf"
    gf.write(path, [("general.alignment", gf.U32, 0)], [])
    _, e = our_read(q8rt, path)
    assert e.endswith("general.alignment is 0"), e


def test_truncated_data_refused_before_upload(q8rt, ref_gguf, tmp_path):
    """A file shorter than its tensor table: the header reads (both readers agree on the shortfall)
    and the upload refuses it before touching the GPU."""
    keys, tensors, _ = gf.model(5, {"token_embd.weight": (64, 256)})
    blob, info = gf.build(keys, tensors)
    path = tmp_path / "short.gguf"
    path.write_bytes(blob[:-100])
    ours, _ = our_read(q8rt, path)
    ref, _ = ref_read(ref_gguf, path)
    assert ours[0] == ref[0] and ours[0]["need"] - ours[0]["file_size"] == 100
    lib = q8rt.load()
    g = q8rt.GGUF(path)
    err = C.create_string_buffer(512)
    assert lib.rt_gguf_upload(None, C.byref(g.h), os.fsencode(path), err, 512) == -1
    assert "truncated: the file is 100 B short of its tensor table" in err.value.decode()
    g.close()


def test_model_writer_round_trip(q8rt, tmp_path):
    """The qwen35-like model file the GPU tests upload: its Q8_0 bytes are where the table says."""
    shapes = {"token_embd.weight": (64, 256), "blk.0.ffn_gate.weight": (96, 256), "blk.0.ffn_down.weight": (256, 96)}
    keys, tensors, q8 = gf.model(11, shapes)
    path = tmp_path / "m.gguf"
    gf.write(path, keys, tensors)
    raw = np.fromfile(path, np.uint8)
    with q8rt.GGUF(path) as g:
        for name, (rows, cols) in shapes.items():
            t = g.tensor(name)
            assert t["dim"][:2] == [cols, rows] and t["bytes"] == rows * cols // 32 * 34
            assert np.array_equal(raw[t["offset"]:t["offset"] + t["bytes"]], q8[name])


def test_upload_refuses_bad_shapes_before_the_gpu(q8rt, tmp_path):
    """Q8_0 tensors the products cannot take are refused with their name before anything is
    uploaded, so no GPU is needed to see it: a 1-D tensor, dimensions whose product overflows 64
    bits, and more than 2^32 rows (each alone in its file)."""
    lib = q8rt.load()
    cases = [("vec", [256], "is not a matrix"), ("huge", [32, 2**40, 2**40], "out of range"), ("tall", [32, 2**33], "out of range")]
    for name, dims, want in cases:
        path = tmp_path / f"{name}.gguf"
        # a header naming the tensor, with no data: the size check must not be what refuses it
        head = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + gf.gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gf.Q8_0, 0)
        path.write_bytes(head)
        g = q8rt.GGUF(path)
        # make the file "complete" as far as the table says, so that the shape is what fails
        g.h.need = g.h.file_size
        err = C.create_string_buffer(512)
        assert lib.rt_gguf_upload(None, C.byref(g.h), os.fsencode(path), err, 512) == -1
        assert f"tensor {name}:" in err.value.decode() and want in err.value.decode(), err.value.decode()
        g.close()


@pytest.mark.parametrize("vt,v", [(gf.STR, "64"), (gf.F32, 64.0), (gf.U64, 64), (gf.I32, 64), (gf.U8, 64), (gf.F64, 64.0)])
def test_alignment_of_any_type_read_as_the_reference(q8rt, tmp_path, vt, v):
    """general.alignment is read as the reference reads it, strtoull of the key's text
    (gguf_reader.c:198-202), whatever the key's type: 64 as a string, a float or any integer type
    puts the data on the writer's 64-byte boundary, as the reference's reader does."""
    keys = [("general.architecture", gf.STR, "qwen35"), ("general.alignment", vt, v)]
    path = tmp_path / "a.gguf"
    info = gf.write(path, keys, TENSORS_ALL, alignment=64)
    ours, e = our_read(q8rt, path)
    assert e is None, e
    assert ours[0]["data_start"] == info["data_start"] and info["data_start"] % 64 == 0
    assert [t["offset"] for t in ours[2]] == [info["offsets"][t["name"]] for t in TENSORS_ALL]


def test_alignment_of_any_type_matches_reference_reader(q8rt, ref_gguf, tmp_path):
    for i, (vt, v) in enumerate([(gf.STR, "64"), (gf.F32, 64.0), (gf.I16, 64), (gf.STR, "4096")]):
        keys = [("general.architecture", gf.STR, "qwen35"), ("general.alignment", vt, v)]
        path = tmp_path / f"a{i}.gguf"
        gf.write(path, keys, TENSORS_ALL, alignment=int(float(v)))
        ours, e1 = our_read(q8rt, path)
        ref, e2 = ref_read(ref_gguf, path)
        assert e1 is None and e2 is None, (e1, e2)
        assert ours[0] == ref[0] and ours[2] == ref[2], (vt, v)


def _raw_header(offset, alignment_key=None):
    """GGUF v3 bytes: optionally a general.alignment key (type, value), then one Q8_0 tensor of 16 x 32
    (544 bytes) at the given offset from the data start; a little data after the header."""
    nkeys = 1 if alignment_key else 0
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, nkeys)
    if alignment_key:
        head += gf.key("general.alignment", *alignment_key)
    head += gf.gstr("blk.0.w.weight") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 16) + struct.pack("<IQ", gf.Q8_0, offset)
    return head + bytes(64)


@pytest.mark.parametrize("offset", [2**64 - 32, 2**64 - 544])
def test_offset_past_2_64_refused(q8rt, tmp_path, offset):
    """A tensor whose offset + size wraps 64 bits (the reference's sums would wrap and pass its size
    checks) is refused with the tensor's name."""
    path = tmp_path / "wrap.gguf"
    path.write_bytes(_raw_header(offset))
    _, e = our_read(q8rt, path)
    assert e is not None and "blk.0.w.weight" in e and "overflows 64 bits" in e, e


def test_data_end_past_2_64_refused(q8rt, tmp_path):
    """An offset whose end fits in 64 bits (2^64 - 32) but lands past 2^64 once the data start (96
    here) is added is refused."""
    path = tmp_path / "wrap2.gguf"
    path.write_bytes(_raw_header(2**64 - 576))
    _, e = our_read(q8rt, path)
    assert e is not None and "past 2^64 bytes" in e, e


@pytest.mark.parametrize("key", [(gf.I8, -1), (gf.I64, -32), (gf.U64, 2**64 - 1)])
def test_alignment_past_2_64_refused(q8rt, tmp_path, key):
    """A negative alignment key reads, as strtoull reads "-1", as 2^64 - 1: the data start would wrap,
    so the file is refused."""
    path = tmp_path / "al.gguf"
    path.write_bytes(_raw_header(0, key))
    _, e = our_read(q8rt, path)
    assert e is not None and "general.alignment" in e and "past 2^64 bytes" in e, e
