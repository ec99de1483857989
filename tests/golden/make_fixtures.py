"""Writes tests/golden/ref_products.npz: outputs of the reference's own Q8_0 products, compiled from
its sources (src/card/gemv.c, gemm.c, knc.h host model) into oracle/_ref/libref.so by oracle/Makefile,
on small seeded cases. Every y is the reference's gemv_i_thread / gemm_i_thread at one thread
(whole groups), bit for bit. Inputs are stored with the outputs, except config 1's 4096x4096 matrix,
which is regenerated from seed 0 by tests/synth.py and checked against the stored SHA-256.

Run in the build container (where /root/reference exists): python tests/golden/make_fixtures.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import synth  # noqa: E402
from oracle_ffi import Reference  # noqa: E402

# (seed, rows, cols, t, dist): t crosses every token chunk of gemm.c (8, 4, 3, 2, 1) and the
# pass size (16); cols from one block to 16; rows from one group to 4.
CASES = [
    (1, 16, 32, 1, "normal"),
    (2, 16, 96, 3, "normal"),
    (3, 32, 512, 1, "normal"),
    (4, 64, 512, 2, "normal"),
    (5, 64, 512, 4, "normal"),
    (6, 48, 256, 5, "normal"),
    (7, 16, 512, 8, "normal"),
    (8, 16, 512, 9, "normal"),
    (9, 32, 256, 16, "normal"),
    (10, 16, 512, 17, "normal"),
    (11, 64, 512, 3, "lognormal"),
    (12, 16, 1024, 40, "normal"),
]


def main():
    ref = Reference()
    out = {}
    for i, (seed, rows, cols, t, dist) in enumerate(CASES):
        q8, x = synth.case(seed, rows, cols, t, dist)
        y = ref.gemm(q8, rows, cols, x)
        for k in range(t):  # gemm == gemv per token, as the reference's own gate holds (scripts/check.sh:132-149)
            assert np.array_equal(ref.gemv(q8, rows, cols, x[k]).view(np.uint32), y[k].view(np.uint32))
        out[f"c{i}_meta"] = np.array([seed, rows, cols, t, dist == "lognormal"], np.int64)
        out[f"c{i}_q8"] = q8
        out[f"c{i}_x"] = x
        out[f"c{i}_y"] = y
    # config 1: y = W x, W 4096x4096, seed 0
    q8, x = synth.case(0, 4096, 4096, 1)
    out["cfg1_y"] = ref.gemv(q8, 4096, 4096, x[0])
    out["cfg1_sha_q8"] = np.frombuffer(hashlib.sha256(q8.tobytes()).digest(), np.uint8)
    out["cfg1_sha_x"] = np.frombuffer(hashlib.sha256(x.tobytes()).digest(), np.uint8)
    out["ncases"] = np.array([len(CASES)])
    np.savez_compressed(os.path.join(HERE, "ref_products.npz"), **out)
    print("wrote", os.path.join(HERE, "ref_products.npz"), sum(v.nbytes for v in out.values()), "bytes raw")


if __name__ == "__main__":
    main()
