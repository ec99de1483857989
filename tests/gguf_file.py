"""Synthetic GGUF v3 files for the tests, written from the published format (ggml's gguf.md):
"GGUF", u32 version, u64 tensor count, u64 key count; keys (u64-length UTF-8 name, u32 value type,
value; an array is u32 element type, u64 count, elements); tensor infos (name, u32 dimension count,
u64 dims ne0 first, u32 ggml type, u64 offset from the data start, a multiple of the alignment);
zero padding to general.alignment (32 when absent); the data.

The writer also makes the malformed files the error tests need (a wrong magic, a header cut short,
a bad type), and records where each part of the header ended, so a test can check the reader's
offsets against the bytes actually written.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
PACK = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}
Q8_0, F32_T, F16_T, Q4_0 = 8, 0, 1, 2
# ggml types the tests use: (elements a block, bytes a block)
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 30: (1, 2)}


def gstr(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(vt, v):
    if vt == STR:
        return gstr(v)
    return struct.pack(PACK[vt], v)


def key(name, vt, v):
    """One key: for vt == ARR, v = (element type, [elements])."""
    out = gstr(name) + struct.pack("<I", vt)
    if vt == ARR:
        et, items = v
        out += struct.pack("<IQ", et, len(items)) + b"".join(value(et, i) for i in items)
    else:
        out += value(vt, v)
    return out


def tensor_bytes(dims, ggml_type):
    n = int(np.prod(dims, dtype=np.uint64))
    blk, size = BLOCK[ggml_type]
    return n // blk * size


def build(keys, tensors, alignment=32, version=3, magic=b"GGUF"):
    """The file as bytes, and a dict of where things are.

    keys: [(name, vt, value)]; tensors: [dict(name, dims, type, data=bytes or None, tie=name)].
    A tensor with `tie` gets the offset of the named earlier tensor and no data of its own; one
    with data None gets zeros. Offsets are laid out in order, each a multiple of `alignment`."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(keys))
    head += b"".join(key(*k) for k in keys)
    keys_end = len(head)
    offsets, blobs, at = {}, [], 0
    for t in tensors:
        nbytes = tensor_bytes(t["dims"], t["type"])
        if t.get("tie"):
            offsets[t["name"]] = offsets[t["tie"]]
            continue
        at = (at + alignment - 1) // alignment * alignment
        offsets[t["name"]] = at
        data = t.get("data")
        data = bytes(nbytes) if data is None else bytes(data)
        assert len(data) == nbytes, (t["name"], len(data), nbytes)
        blobs.append((at, data))
        at += nbytes
    for t in tensors:
        head += gstr(t["name"]) + struct.pack("<I", len(t["dims"])) + b"".join(struct.pack("<Q", d) for d in t["dims"])
        head += struct.pack("<IQ", t["type"], offsets[t["name"]])
    header_end = len(head)
    data_start = (header_end + alignment - 1) // alignment * alignment
    body = bytearray(at)
    for off, data in blobs:
        body[off:off + len(data)] = data
    blob = head + bytes(data_start - header_end) + bytes(body)
    info = {"keys_end": keys_end, "header_end": header_end, "data_start": data_start,
            "offsets": {n: data_start + o for n, o in offsets.items()}, "size": len(blob)}
    return blob, info


def write(path, keys, tensors, alignment=32, **kw):
    blob, info = build(keys, tensors, alignment=alignment, **kw)
    with open(path, "wb") as f:
        f.write(blob)
    return info


def model(seed, shapes, extra_keys=(), alignment=32, tie_output=True):
    """A small qwen35-like file: Q8_0 matrices {name: (rows, cols)} with seeded synthetic rows, an F32
    norm, and (tie_output) output.weight tied to token_embd.weight by offset. Returns (keys, tensors,
    {name: q8 bytes})."""
    import synth

    rng = np.random.default_rng(seed)
    keys = [("general.architecture", STR, "qwen35"), ("qwen35.block_count", U32, 1)]
    if alignment != 32:
        keys.append(("general.alignment", U32, alignment))
    keys += list(extra_keys)
    tensors, q8 = [], {}
    for name, (rows, cols) in shapes.items():
        q8[name] = synth.q8_rows(rng, rows, cols)
        tensors.append({"name": name, "dims": [cols, rows], "type": Q8_0, "data": q8[name].tobytes()})
    cols0 = next(iter(shapes.values()))[1]
    norm = rng.standard_normal(cols0).astype(np.float32)
    tensors.append({"name": "output_norm.weight", "dims": [cols0], "type": F32_T, "data": norm.tobytes()})
    if tie_output and "token_embd.weight" in shapes:
        rows, cols = shapes["token_embd.weight"]
        tensors.append({"name": "output.weight", "dims": [cols, rows], "type": Q8_0, "tie": "token_embd.weight"})
    return keys, tensors, q8
