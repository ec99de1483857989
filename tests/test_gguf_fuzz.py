"""The GGUF header reader (intel-phi-apl_amd/csrc/q8_gguf.cpp) under seeded corruption, on the CPU.

tests/c/gguf_fuzz.cpp is built with AddressSanitizer and UndefinedBehaviorSanitizer around the
reader's own source and reads a few thousand files made from valid ones (every key type, arrays,
strings, Q8_0 and F32 tensors, a tie, alignments 32 and 64): bytes flipped in the header, 4- and
8-byte fields set to extreme counts, lengths, types and offsets, the file cut short, bytes inserted
or repeated. Every file must be accepted or refused without a sanitizer report, a refusal must say
"path: reason", and an accepted header must keep its invariants (the harness's checks). The
reader's known-answer and reference comparisons are in tests/test_gguf.py."""
import os
import struct
import subprocess

import numpy as np
import pytest

import gguf_file as gf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INTERESTING_64 = [0, 1, 2, 31, 32, 33, 4096, 2**31, 2**32 - 1, 2**32, 2**62, 2**63, 2**64 - 32, 2**64 - 1]
INTERESTING_32 = [0, 1, 4, 5, 8, 12, 13, 14, 42, 43, 0x7FFFFFFF, 0xFFFFFFFF]


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("fuzz") / "gguf_fuzz")
    subprocess.run(["g++", "-O1", "-g", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
                    "-fno-omit-frame-pointer", "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "intel-phi-apl_amd", "csrc", "q8_gguf.cpp"),
                    os.path.join(ROOT, "tests", "c", "gguf_fuzz.cpp"), "-o", exe], check=True)
    return exe


def seeds():
    """Valid files as bytes, with where each header ends."""
    out = []
    keys = [("general.architecture", gf.STR, "qwen35"), ("a.u8", gf.U8, 255), ("a.i8", gf.I8, -128), ("a.u16", gf.U16, 65535),
            ("a.i16", gf.I16, -32768), ("a.u32", gf.U32, 2**32 - 1), ("a.i32", gf.I32, -2**31), ("a.f32", gf.F32, 1.5),
            ("a.bool", gf.BOOL, 1), ("a.u64", gf.U64, 2**64 - 1), ("a.i64", gf.I64, -2**63), ("a.f64", gf.F64, -0.25),
            ("a.arr_u32", gf.ARR, (gf.U32, [1, 2, 3])), ("a.arr_str", gf.ARR, (gf.STR, ["x", "yz"])), ("a.long_str", gf.STR, "s" * 300)]
    tensors = [{"name": "token_embd.weight", "dims": [64, 32], "type": gf.Q8_0}, {"name": "norm.weight", "dims": [64], "type": gf.F32_T},
               {"name": "output.weight", "dims": [64, 32], "type": gf.Q8_0, "tie": "token_embd.weight"},
               {"name": "cube", "dims": [32, 2, 2, 2], "type": gf.Q8_0}]
    for alignment in (32, 64):
        blob, info = gf.build(keys + ([("general.alignment", gf.U32, alignment)] if alignment != 32 else []), tensors, alignment=alignment)
        out.append((blob, info["header_end"]))
    blob, info = gf.build([("general.alignment", gf.STR, "64")], [{"name": "w", "dims": [32, 16], "type": gf.Q8_0}], alignment=64)
    out.append((blob, info["header_end"]))
    blob, info = gf.build([], [])
    out.append((blob, info["header_end"]))
    return out


def mutate(rng, blob, header_end):
    b = bytearray(blob)
    for _ in range(int(rng.integers(1, 4))):
        op = int(rng.integers(0, 6))
        span = max(1, min(len(b), header_end + 8))
        if op == 0 and b:  # flip bytes in the header
            for _ in range(int(rng.integers(1, 5))):
                i = int(rng.integers(0, span))
                b[i] ^= int(rng.integers(1, 256))
        elif op == 1 and len(b) >= 8:  # an extreme 8-byte field
            i = int(rng.integers(0, max(1, min(span, len(b) - 8))))
            b[i:i + 8] = struct.pack("<Q", INTERESTING_64[int(rng.integers(0, len(INTERESTING_64)))])
        elif op == 2 and len(b) >= 4:  # an extreme 4-byte field
            i = int(rng.integers(0, max(1, min(span, len(b) - 4))))
            b[i:i + 4] = struct.pack("<I", INTERESTING_32[int(rng.integers(0, len(INTERESTING_32)))])
        elif op == 3:  # cut short
            b = b[:int(rng.integers(0, len(b) + 1))]
        elif op == 4:  # insert bytes
            i = int(rng.integers(0, len(b) + 1))
            b[i:i] = rng.integers(0, 256, int(rng.integers(1, 9))).astype(np.uint8).tobytes()
        elif b:  # repeat a chunk
            i = int(rng.integers(0, len(b)))
            n = int(rng.integers(1, 33))
            b[i:i] = b[i:i + n]
    return bytes(b)


@pytest.mark.parametrize("seed", [1, 2])
def test_reader_survives_corrupted_files(fuzzer, tmp_path, seed):
    rng = np.random.default_rng(seed)
    base = seeds()
    paths = []
    for i, (blob, header_end) in enumerate(base):  # the valid files themselves are accepted
        p = tmp_path / f"valid{i}.gguf"
        p.write_bytes(blob)
        paths.append(str(p))
    for i in range(2000):
        blob, header_end = base[int(rng.integers(0, len(base)))]
        p = tmp_path / f"m{i}.gguf"
        p.write_bytes(mutate(rng, blob, header_end))
        paths.append(str(p))
    lst = tmp_path / "list.txt"
    lst.write_text("\n".join(paths) + "\n")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([fuzzer, str(lst)], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
    acc, ref = (int(v) for v in r.stdout.split()[1:4:2])
    assert acc >= len(base) and ref > 0 and acc + ref == len(paths), r.stdout
