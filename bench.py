#!/usr/bin/env python3
"""Benchmark of the Q8_0 weight products on one MI355X.

The step is one 9B-class decode token at M = 1: 32 layers of
    QKV 6144x4096, out 4096x4096, gate+up 2 x 12288x4096 fused into SiLU(g)*u, down 4096x12288,
then the output head 151936x4096: 129 products, 7,230,391,808 B of Q8_0 weights resident in HBM
(distinct per layer, synthetic: q uniform in [-127, 127], d = binary16(|N(0, 0.02)|/127)), every
byte streamed once per token. Activations are already in HBM. The token is recorded once as a
HIP graph and replayed.

value = algorithmic bytes per token (Q8_0 weights + x read once + y written once, per product)
        x tokens / time, in GB/s; ms_per_step = ms per token.
roofline = the dominant kernel (the fused gate+up): its algorithmic bytes per launch over its
        average duration, from events attached to each of its launches in a timed replay.
cpu_baseline = the reference's own host path (oracle/_ref: src/card/gemv.c with the team of
        src/card/team.c, built from the reference's sources with its own host flags) on this
        host's cores, over one 9B layer's five products; the oracle's own restatement when
        oracle/_ref is absent. Beside it, under cpu_baseline.configs, the same path on the
        4096x4096 GEMV, the M = 16 GEMM and the M = 4 verify products, and under
        cpu_baseline.variants the layer on the build with -mfma added.

Also in the line, each measured with its own weights rotated through >= 512 MB so that the
256 MB Infinity Cache cannot serve them: the single 4096x4096 GEMV, the draft head (first 32768
rows), the prompt GEMM at M = 16, 40 and 64, the verify path at M = 2..4 (fused pair + down,
heavy-tailed scales), the 2B layer set, the DeltaNet quartet as four launches and as one round,
a 9B layer with its norm and residual epilogues, the host-pointer entry points and the whole 9B
token through them (PCIe-inclusive, timed from C by intel-phi-apl_amd/q8_hostbench), and the GGUF
load of one 9B layer. Each of these runs in a process of its own before the token, on fresh device
memory as the token's weights are. Beside the token: the floor token, the same 129 positions as
pure reads on the products' own grids (rt_q8_read_dev), one graph.
"""
import argparse
import ctypes as c
import importlib.util
import json
import os
import statistics
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
MALL_ROTATE_BYTES = 512 << 20

HIDDEN, FFN, QKV, VOCAB, DRAFT, LAYERS = 4096, 12288, 4096 + 2 * 1024, 151936, 32768, 32


def package():
    spec = importlib.util.spec_from_file_location("q8rt", os.path.join(ROOT, "intel-phi-apl_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["q8rt"] = mod
    spec.loader.exec_module(mod)
    return mod


def q8_bytes(rows, cols):
    return rows * cols // 32 * 34


def alg_bytes(rows, cols, t, pair=False):
    """Weights once, x once, y once (the fused pair: both weights, x once, SiLU(g)*u once)."""
    return q8_bytes(rows, cols) * (2 if pair else 1) + 4 * t * cols + 4 * t * rows


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Bench:
    def __init__(self, q8rt):
        self.q8rt = q8rt
        self.rt = q8rt.Runtime()
        self.lib, self.R = self.rt.lib, self.rt.R
        self.staging = self.rt.alloc(q8_bytes(VOCAB, HIDDEN))
        self.seed = 1000
        self.knames = {}

    def matrix(self, rows, cols, dist=0, mu=0.0, sigma=0.02):
        """Synthetic GGUF rows drawn on the GPU, repacked to the device form: a resident handle."""
        self.seed += 1
        w = self.rt.alloc(q8_bytes(rows, cols))
        self.lib.rt_q8_fill_dev(self.R, c.c_void_p(self.staging), rows, cols, self.seed, dist, mu, sigma)
        self.lib.rt_q8_repack_dev(self.R, c.c_void_p(self.staging), rows, cols, c.c_void_p(w))
        return w

    def vec(self, n):
        self.seed += 1
        p = self.rt.alloc(4 * n)
        self.lib.rt_f32_fill_dev(self.R, c.c_void_p(p), n, self.seed)
        return p

    def gemm(self, w, rows, cols, x, t, y, xs=None):
        self.lib.rt_gemm_dev(self.R, c.c_void_p(w), rows, cols, c.c_void_p(x), xs or cols, t, c.c_void_p(y))

    def pair(self, wg, wu, rows, cols, x, t, y):
        self.lib.rt_gemv_swiglu_dev(self.R, c.c_void_p(wg), c.c_void_p(wu), rows, cols, c.c_void_p(x), cols, t, c.c_void_p(y))

    def timed(self, fn, reps):
        self.rt.sync()
        self.lib.rt_timer_start(self.R)
        for _ in range(reps):
            fn()
        return self.lib.rt_timer_stop(self.R) / reps

    def ktimes(self, fn, reps):
        """Per-launch kernel durations (us) of every product fn makes, by (kind, rows, cols, t); the
        kernel's name and grid (threads) as rocprof reports them in self.knames[(kind, rows, cols, t)]."""
        self.lib.rt_ktime(self.R, 1)
        for _ in range(reps):
            fn()
        n = 16384
        kind, rows, cols, t = (np.zeros(n, np.int32), np.zeros(n, np.int64), np.zeros(n, np.int64), np.zeros(n, np.int64))
        us, grid = np.zeros(n, np.float32), np.zeros(n, np.int64)
        names = c.create_string_buffer(64 * n)
        got = self.lib.rt_ktime_read(self.R, *(self.q8rt.ptr(a) for a in (kind, rows, cols, t, us)), names, self.q8rt.ptr(grid), n)
        self.lib.rt_ktime(self.R, 0)
        out = {}
        for i in range(got):
            key = (self.q8rt.KINDS[int(kind[i])], int(rows[i]), int(cols[i]), int(t[i]))
            out.setdefault(key, []).append(float(us[i]))
            self.knames[key] = (names.raw[64 * i:64 * i + 64].split(b"\0")[0].decode(), int(grid[i]))
        return out


def rotation(bench, rows, cols, copies_min=2, **kw):
    per = q8_bytes(rows, cols)
    n = max(copies_min, -(-MALL_ROTATE_BYTES // per))
    return [bench.matrix(rows, cols, **kw) for _ in range(n)]


def token_9b(b):
    """The 9B decode token's weights (distinct per layer) and activations, and the token as a function
    that enqueues its 129 products; and its algorithmic bytes."""
    log(f"9B decode: {LAYERS} layers + head, {7230391808 / 1e9:.2f} GB of Q8_0 weights")
    layers = [dict(qkv=b.matrix(QKV, HIDDEN), out=b.matrix(HIDDEN, HIDDEN), gate=b.matrix(FFN, HIDDEN), up=b.matrix(FFN, HIDDEN),
                   down=b.matrix(HIDDEN, FFN)) for _ in range(LAYERS)]
    head = b.matrix(VOCAB, HIDDEN)
    xh, xa, h = b.vec(HIDDEN), b.vec(HIDDEN), b.vec(FFN)
    yq, yo, yd, logits = b.vec(QKV), b.vec(HIDDEN), b.vec(HIDDEN), b.vec(VOCAB)

    def token():
        for L in layers:
            b.gemm(L["qkv"], QKV, HIDDEN, xh, 1, yq)
            b.gemm(L["out"], HIDDEN, HIDDEN, xa, 1, yo)
            b.pair(L["gate"], L["up"], FFN, HIDDEN, xh, 1, h)
            b.gemm(L["down"], HIDDEN, FFN, h, 1, yd)
        b.gemm(head, VOCAB, HIDDEN, xh, 1, logits)

    sink = b.vec(VOCAB)  # a word a workgroup of the largest grid
    V = c.c_void_p

    def floor():
        """the same 129 positions, each the product's loads on its grid and nothing else (rt_q8_read_dev)"""
        for L in layers:
            b.lib.rt_q8_read_dev(b.R, V(L["qkv"]), None, QKV, HIDDEN, V(xh), HIDDEN, 1, V(sink))
            b.lib.rt_q8_read_dev(b.R, V(L["out"]), None, HIDDEN, HIDDEN, V(xa), HIDDEN, 1, V(sink))
            b.lib.rt_q8_read_dev(b.R, V(L["gate"]), V(L["up"]), FFN, HIDDEN, V(xh), HIDDEN, 1, V(sink))
            b.lib.rt_q8_read_dev(b.R, V(L["down"]), None, HIDDEN, FFN, V(h), FFN, 1, V(sink))
        b.lib.rt_q8_read_dev(b.R, V(head), None, VOCAB, HIDDEN, V(xh), HIDDEN, 1, V(sink))

    token.floor = floor
    per_token = LAYERS * (alg_bytes(QKV, HIDDEN, 1) + alg_bytes(HIDDEN, HIDDEN, 1) + alg_bytes(FFN, HIDDEN, 1, pair=True) +
                          alg_bytes(HIDDEN, FFN, 1)) + alg_bytes(VOCAB, HIDDEN, 1)
    return layers, head, token, per_token


TRACE_REPLAYS = 20


def token_trace(b):
    """The 9B token as one graph replayed TRACE_REPLAYS times, each replay alone on the GPU (the
    stream idle before and after it), then launched eagerly as many times the same way, after one
    untimed replay and one untimed eager token. Under rocprofv3 --kernel-trace every kernel of every
    replay has its begin and end, so summarize_trace gives each of the 129 kernels of a replay its
    duration and the gap from its end to the next kernel's begin. Also each replay's own time on the
    stream's events, beside the trace's."""
    layers, head, token, per_token = token_9b(b)
    graphs = []
    for fn in (token, token.floor):
        b.lib.rt_graph_begin(b.R)
        fn()
        graphs.append(b.lib.rt_graph_end(b.R))
    run = lambda: b.lib.rt_graph_launch(b.R, c.c_void_p(graphs[0]))  # noqa: E731
    run_floor = lambda: b.lib.rt_graph_launch(b.R, c.c_void_p(graphs[1]))  # noqa: E731
    out = {"replays": TRACE_REPLAYS, "products": 4 * LAYERS + 1, "bytes_per_token": per_token}
    for key, fn in (("graph", run), ("eager", token), ("floor", run_floor)):
        fn()
        b.rt.sync()
        ms = []
        for _ in range(TRACE_REPLAYS):
            ms.append(b.timed(fn, 1))
        out[key] = {"ms_median": round(statistics.median(ms), 4), "ms_min": round(min(ms), 4)}
        log(f"  {key}: {out[key]}")
    for g in graphs:
        b.lib.rt_graph_free(b.R, c.c_void_p(g))
    for L in layers:
        for w in L.values():
            b.rt.free(w)
    b.rt.free(head)
    return out


def decode_9b(b, steps, warmup):
    layers, head, token, per_token = token_9b(b)
    b.lib.rt_graph_begin(b.R)
    token()
    graph = b.lib.rt_graph_end(b.R)
    run = lambda: b.lib.rt_graph_launch(b.R, c.c_void_p(graph))  # noqa: E731
    # settle, untimed, before the warmup steps: replays in groups of 10 for at least 150 ms, so that the
    # timed steps start from the GPU's steady state whatever the warmup count (with 5 warmup steps and
    # no settle, one run in two timed 20 steps 3.5 % slower: 1.470 against 1.420 ms a token)
    t0, b.settle_replays = time.perf_counter(), 0
    while time.perf_counter() - t0 < 0.15:
        for _ in range(10):
            run()
        b.rt.sync()
        b.settle_replays += 10
    for _ in range(warmup):
        run()
    ms_graph = b.timed(run, steps)
    ms_eager = b.timed(token, max(1, steps // 4))
    log(f"  token: graph {ms_graph:.3f} ms, eager {ms_eager:.3f} ms")
    # the floor: the same 129 positions as pure reads on the products' grids, one graph
    b.lib.rt_graph_begin(b.R)
    token.floor()
    fgraph = b.lib.rt_graph_end(b.R)
    frun = lambda: b.lib.rt_graph_launch(b.R, c.c_void_p(fgraph))  # noqa: E731
    for _ in range(max(warmup, 5)):
        frun()
    b.floor_ms = b.timed(frun, steps)
    b.floor_kernels = {}
    for (kind, rows, cols, t), v in sorted(b.ktimes(token.floor, min(steps, 100)).items()):
        b.floor_kernels[f"{kind} {rows}x{cols} t{t}"] = round(statistics.fmean(v), 3)
    b.lib.rt_graph_free(b.R, c.c_void_p(fgraph))
    log(f"  floor (pure reads on the same grids): graph {b.floor_ms:.3f} ms; {b.floor_kernels}")
    kt = b.ktimes(token, min(steps, 100))
    b.lib.rt_graph_free(b.R, c.c_void_p(graph))
    kernels = {}
    for (kind, rows, cols, t), v in sorted(kt.items()):
        pair = kind.endswith("pair")
        mean = statistics.fmean(v)
        gbs = alg_bytes(rows, cols, t, pair) / mean / 1e3
        kname, grid = b.knames[(kind, rows, cols, t)]
        kernels[f"{kind} {rows}x{cols} t{t}"] = {"us": round(mean, 3), "GB/s": round(gbs, 1), "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
                                                 "floor_us": b.floor_kernels.get(f"{kind} {rows}x{cols} t{t}"),
                                                 "launches": len(v), "kernel": kname, "grid": grid, "alg_bytes": alg_bytes(rows, cols, t, pair)}
        log(f"  {kind:9s} {rows:6d}x{cols:<5d} t{t}: {mean:8.2f} us  {gbs:7.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM)")
    # the dominant kernel: the most time per token
    dom = max(kt.items(), key=lambda kv: statistics.fmean(kv[1]) * len(kv[1]))
    (kind, rows, cols, t), v = dom
    per_launch = alg_bytes(rows, cols, t, kind.endswith("pair"))
    mean_us = statistics.fmean(v)
    kname, grid = b.knames[(kind, rows, cols, t)]
    roof = {"kernel": f"{kname} ({kind} {rows}x{cols}, t={t}, grid {grid})", "bound": "hbm",
            "achieved": round(per_launch / mean_us / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(per_launch / mean_us / 1e3 / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(kname, grid),
            "traffic_source": os.path.relpath(DECODE_PROFILE, ROOT) + " (rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by the copy kernel)",
            "bytes_per_launch": per_launch,
            "us_per_launch": round(mean_us, 3), "launches_timed": len(v)}
    return per_token, ms_graph, ms_eager, kernels, roof, layers


def read_floor_us(b, ws, rows, cols, x, t=1):
    """Mean duration of the pure read of each rotated copy on its product's grid at t tokens
    (rt_q8_read_dev; x holds t rows of cols floats): the floor the product's kernel is held against."""
    sink = b.vec(rows)
    V = c.c_void_p
    reads = lambda: [b.lib.rt_q8_read_dev(b.R, V(w), None, rows, cols, V(x), cols, t, V(sink)) for w in ws]  # noqa: E731
    reads()
    return statistics.fmean(next(iter(b.ktimes(reads, 4).values())))


def single_gemv(b):
    """Config 1's shape on the GPU: 4096x4096, rotated through >= 512 MB of copies, and its floor."""
    ws = rotation(b, 4096, 4096)
    x, y = b.vec(4096), b.vec(4096)
    [b.gemm(w, 4096, 4096, x, 1, y) for w in ws]  # one untimed pass: the copies' first touch and the kernel's first launch
    kt = b.ktimes(lambda: [b.gemm(w, 4096, 4096, x, 1, y) for w in ws], 4)
    us = statistics.fmean(next(iter(kt.values())))
    ms = b.timed(lambda: [b.gemm(w, 4096, 4096, x, 1, y) for w in ws], 4) / len(ws)
    floor = read_floor_us(b, ws, 4096, 4096, x)
    for w in ws:
        b.rt.free(w)
    gb = alg_bytes(4096, 4096, 1)
    return {"kernel_us": round(us, 3), "GB/s": round(gb / us / 1e3, 1), "back_to_back_us": round(1e3 * ms, 3), "floor_us": round(floor, 3),
            "copies": len(ws)}


def draft_head(b):
    ws = rotation(b, DRAFT, HIDDEN)
    x, y = b.vec(HIDDEN), b.vec(DRAFT)
    [b.gemm(w, DRAFT, HIDDEN, x, 1, y) for w in ws]  # one untimed pass
    kt = b.ktimes(lambda: [b.gemm(w, DRAFT, HIDDEN, x, 1, y) for w in ws], 4)
    us = statistics.fmean(next(iter(kt.values())))
    kname, grid = b.knames[next(iter(kt))]
    floor = read_floor_us(b, ws, DRAFT, HIDDEN, x)
    for w in ws:
        b.rt.free(w)
    gb = alg_bytes(DRAFT, HIDDEN, 1)
    return {"rows": DRAFT, "kernel_us": round(us, 3), "GB/s": round(gb / us / 1e3, 1), "floor_us": round(floor, 3), "copies": len(ws), "kernel": kname,
            "grid": grid}


def prompt_gemm(b):
    """Config 4: Y = X W^T, M = 16 and 40 (and 64), on gate/up 12288x4096 and down 4096x12288.

    product_us: the whole product (the matrix-core kernel and, with a K split, the kernel adding
    the partials) back to back over the rotated copies, stream events; GFLOPS and GB/s are over
    it. kernel_us: the matrix-core kernel alone (events on its launch). GFLOPS counts
    2*M*rows*cols; mfma_util_kernel is the bf16 MFMA work actually issued (three limbs, tokens
    padded to 16) over the matrix-core kernel's time, against the dense bf16 peak. floor_us (M =
    16): the x-resident kernel's own loads on its grid with no arithmetic (rt_q8_read_dev at 16
    tokens). Timed after one untimed pass over the copies."""
    out = {}
    for rows, cols in ((FFN, HIDDEN), (HIDDEN, FFN)):
        ws = rotation(b, rows, cols)
        x, y = b.vec(64 * cols), b.vec(64 * rows)
        for m in (16, 40, 64):
            [b.gemm(w, rows, cols, x, m, y) for w in ws]  # one untimed pass (and the workspace sized before timing)
            kt = b.ktimes(lambda: [b.gemm(w, rows, cols, x, m, y) for w in ws], 3)
            us = statistics.fmean([u for v in kt.values() for u in v])
            ms = b.timed(lambda: [b.gemm(w, rows, cols, x, m, y) for w in ws], 3) / len(ws)
            flop = 2.0 * m * rows * cols
            issued = 2.0 * 3 * (16 * -(-m // 16)) * rows * cols
            kname, grid = b.knames[next(iter(kt))]
            out[f"M{m} {rows}x{cols}"] = {"kernel": kname, "grid": grid, "product_us": round(1e3 * ms, 3), "kernel_us": round(us, 3),
                                          "GFLOPS": round(flop / ms / 1e6, 1), "GFLOPS_kernel": round(flop / us / 1e3, 1),
                                          "GB/s": round(alg_bytes(rows, cols, m) / ms / 1e6, 1),
                                          "pct_hbm": round(100 * alg_bytes(rows, cols, m) / ms / 1e6 / HBM_PEAK_GBS, 1),
                                          "mfma_util_kernel": round(issued / us / 1e6 / BF16_PEAK_TFLOPS, 4), "copies": len(ws)}
            if m <= 16:  # the x-resident kernel's loads on its grid, no arithmetic
                out[f"M{m} {rows}x{cols}"]["floor_us"] = round(read_floor_us(b, ws, rows, cols, x, m), 3)
        for w in ws:
            b.rt.free(w)
        b.rt.free(x)
        b.rt.free(y)
    return out


def verify_path(b):
    """Config 5: M = 2..4 tokens, fused gate+up (2 x 12288x4096) then down 4096x12288, d lognormal(ln 0.002, 1),
    over rotated weight sets; each kernel's mean duration (events on its launches) over three passes
    after one untimed pass (the first launches run on cold page tables and code: up to 2x slower),
    and beside it its floor: the same loads at M tokens on the product's own grid, no arithmetic
    (rt_q8_read_dev), timed the same way."""
    kw = dict(dist=1, mu=float(np.log(0.002)), sigma=1.0)
    per = 2 * q8_bytes(FFN, HIDDEN) + q8_bytes(HIDDEN, FFN)
    n = max(2, -(-MALL_ROTATE_BYTES // per))
    sets = [(b.matrix(FFN, HIDDEN, **kw), b.matrix(FFN, HIDDEN, **kw), b.matrix(HIDDEN, FFN, **kw)) for _ in range(n)]
    x, h, y = b.vec(4 * HIDDEN), b.vec(4 * FFN), b.vec(4 * HIDDEN)
    sink = b.vec(FFN)
    V = c.c_void_p
    out = {}
    for m in (2, 3, 4):
        def step():
            for g, u, d in sets:
                b.pair(g, u, FFN, HIDDEN, x, m, h)
                b.gemm(d, HIDDEN, FFN, h, m, y)

        def reads():
            for g, u, d in sets:
                b.lib.rt_q8_read_dev(b.R, V(g), V(u), FFN, HIDDEN, V(x), HIDDEN, m, V(sink))
                b.lib.rt_q8_read_dev(b.R, V(d), None, HIDDEN, FFN, V(h), FFN, m, V(sink))
        reads()
        floor = {k: statistics.fmean(v) for k, v in b.ktimes(reads, 3).items()}
        step()  # one untimed pass: the copies' first touch and the kernels' first launch
        kt = b.ktimes(step, 3)
        res = {}
        for (kind, rows, cols, t), v in kt.items():
            pair = kind.endswith("pair")
            us = statistics.fmean(v)
            kname, grid = b.knames[(kind, rows, cols, t)]
            fl = floor.get((kind, rows, cols, t))
            res["fused_gate_up" if pair else "down"] = {"kernel_us": round(us, 3), "GB/s": round(alg_bytes(rows, cols, t, pair) / us / 1e3, 1),
                                                          "pct_hbm": round(100 * alg_bytes(rows, cols, t, pair) / us / 1e3 / HBM_PEAK_GBS, 1),
                                                          "floor_us": round(fl, 3) if fl else None, "kernel": kname, "grid": grid}
        out[f"M{m}"] = res
    for s in sets:
        for w in s:
            b.rt.free(w)
    return out


def deltanet_round(b):
    """The 9B DeltaNet quartet (QKV 8192x4096, GATE 4096x4096, BETA and ALPHA 32x4096, sharing x;
    src/apl/qwen35.apl:93-96) over 32 layers of distinct weights, recorded as a graph: four launches
    a layer against one round launch a layer (rt_gemv_round_dev)."""
    shapes = [8192, 4096, 32, 32]
    layers = [[b.matrix(r, HIDDEN) for r in shapes] for _ in range(LAYERS)]
    x = b.vec(HIDDEN)
    ys = [b.vec(r) for r in shapes]
    per = LAYERS * sum(alg_bytes(r, HIDDEN, 1) for r in shapes) - LAYERS * 3 * 4 * HIDDEN  # x read once a round
    R = (c.c_long * 4)(*shapes)
    Y = (c.c_void_p * 4)(*ys)
    Ws = [(c.c_void_p * 4)(*L) for L in layers]

    def singles():
        for L in layers:
            for w, r, y in zip(L, shapes, ys):
                b.gemm(w, r, HIDDEN, x, 1, y)

    def rounds():
        for W in Ws:
            b.lib.rt_gemv_round_dev(b.R, 4, W, R, HIDDEN, c.c_void_p(x), HIDDEN, 1, Y)

    out = {"bytes": per}
    for key, fn in (("four_launches", singles), ("one_round", rounds)):
        b.lib.rt_graph_begin(b.R)
        fn()
        g = b.lib.rt_graph_end(b.R)
        b.lib.rt_graph_launch(b.R, c.c_void_p(g))
        ms = b.timed(lambda: b.lib.rt_graph_launch(b.R, c.c_void_p(g)), 20)
        b.lib.rt_graph_free(b.R, c.c_void_p(g))
        out[key] = {"us_per_32_layers": round(1e3 * ms, 2), "GB/s": round(per / ms / 1e6, 1)}
    for L in layers:
        for w in L:
            b.rt.free(w)
    return out


def prompt_rounds(b):
    """At M = 16, 40 and 64 tokens (prompt chunks, a speculative verify), three rounds of products that
    share x, over 32 layers of distinct weights, each recorded as a graph: every product launched
    alone (its matrix-core kernel and its partial sum) against one round a layer
    (rt_gemv_round_dev: one launch for the products, one launch of the sums). The 9B DeltaNet quartet (qwen35.apl:93-96), the attention layer's Q, K and V
    (qwen35.apl:117-119) and the FFN's gate and up (12288 x 4096 each), the last also as the fused
    pair SiLU(X Wg^T) * (X Wu^T) (rt_gemv_swiglu_dev: the round with the SwiGLU in its sums' launch).
    GB/s counts the weights' bytes."""
    out = {}
    for m, name, shapes in [(m, name, shapes) for m in (16, 40, 64) for name, shapes in
                            (("deltanet_quartet", [8192, 4096, 32, 32]), ("attention_qkv", [8192, 1024, 1024]), ("ffn_gate_up", [FFN, FFN]))]:
        n = len(shapes)
        layers = [[b.matrix(r, HIDDEN) for r in shapes] for _ in range(LAYERS)]
        x, ys = b.vec(m * HIDDEN), [b.vec(m * r) for r in shapes]
        R, Y = (c.c_long * n)(*shapes), (c.c_void_p * n)(*ys)
        Ws = [(c.c_void_p * n)(*L) for L in layers]
        per = LAYERS * sum(q8_bytes(r, HIDDEN) for r in shapes)

        def singles():
            for L in layers:
                for w, r, y in zip(L, shapes, ys):
                    b.gemm(w, r, HIDDEN, x, m, y)

        def rounds():
            for W in Ws:
                b.lib.rt_gemv_round_dev(b.R, n, W, R, HIDDEN, c.c_void_p(x), HIDDEN, m, Y)

        def swiglu():  # the FFN's SiLU(X Wg^T) * (X Wu^T) as one call (the round, its sums and the SwiGLU fused)
            for L in layers:
                b.pair(L[0], L[1], FFN, HIDDEN, x, m, ys[0])

        res = {"weight_bytes": per}
        runs = (("products_alone", singles), ("one_round", rounds)) + ((("fused_pair_swiglu", swiglu),) if name == "ffn_gate_up" else ())
        for key, fn in runs:
            fn()  # eager first: the workspace is allocated before the graph records
            b.rt.sync()
            b.lib.rt_graph_begin(b.R)
            fn()
            g = b.lib.rt_graph_end(b.R)
            b.lib.rt_graph_launch(b.R, c.c_void_p(g))
            ms = b.timed(lambda: b.lib.rt_graph_launch(b.R, c.c_void_p(g)), 10)
            b.lib.rt_graph_free(b.R, c.c_void_p(g))
            res[key] = {"us_per_layer": round(1e3 * ms / LAYERS, 2), "GB/s": round(per / ms / 1e6, 1)}
        for L in layers:
            for w in L:
                b.rt.free(w)
        b.rt.free(x)
        for y in ys:
            b.rt.free(y)
        out[f"M{m} {name}"] = res
    return out


HOSTBENCH = os.path.join(ROOT, "intel-phi-apl_amd", "q8_hostbench")


def host_path():
    """The host-pointer entry points the reference's generated code calls (src/card/rt.h:61-72),
    timed from C by intel-phi-apl_amd/q8_hostbench (built by the library's Makefile), in a process
    of its own started before this one touches the GPU: rt_gemv on 4096x4096 (microseconds a call),
    the 9B DeltaNet quartet as rt_gemv_q x 4 + rt_gemv_go, and the whole 9B token through rt_gemv /
    rt_gemv_q + rt_gemv_go (milliseconds a token), each with the calls' phases (x staged, launches,
    wait, y copied out; rt_host_timing). x and y in host memory: the PCIe- and wait-inclusive rate."""
    if not os.path.exists(HOSTBENCH):
        raise SystemExit(f"bench.py: {HOSTBENCH} is not built: run make -C intel-phi-apl_amd")
    p = subprocess.run([HOSTBENCH, "10"], stdout=subprocess.PIPE, text=True, timeout=600)
    if p.returncode != 0:
        raise SystemExit(f"bench.py: {HOSTBENCH} failed (exit {p.returncode})")
    return json.loads(p.stdout.strip().splitlines()[-1])


def epilogues_9b(b):
    """The 9B decode layer with the epilogues around its products (src/apl/qwen35.apl:131-139): QKV
    and the gate+up pair on RMS(x), the output and down products added to the residual stream,
    32 layers recorded as one graph, three ways: the products alone (4 launches a layer), with the
    epilogues fused into them (4), and with the norms and adds as kernels of their own (8,
    rt_set_epi_apart). Weights rotate through 32 layers (7.2 GB), as in the token."""
    eps = 1e-6
    layers = [(b.matrix(QKV, HIDDEN), b.matrix(HIDDEN, HIDDEN), b.matrix(FFN, HIDDEN), b.matrix(FFN, HIDDEN), b.matrix(HIDDEN, FFN))
              for _ in range(LAYERS)]
    x, xa, nw1, nw2, q, h, y = b.vec(HIDDEN), b.vec(HIDDEN), b.vec(HIDDEN), b.vec(HIDDEN), b.vec(QKV), b.vec(FFN), b.vec(HIDDEN)
    L, R, V = b.lib, b.R, c.c_void_p

    def bare():
        for qkv, o, g, u, d in layers:
            b.gemm(qkv, QKV, HIDDEN, x, 1, q)
            b.gemm(o, HIDDEN, HIDDEN, xa, 1, y)
            b.pair(g, u, FFN, HIDDEN, x, 1, h)
            b.gemm(d, HIDDEN, FFN, h, 1, y)

    def with_epilogues():
        for qkv, o, g, u, d in layers:
            L.rt_gemm_norm_dev(R, V(qkv), QKV, HIDDEN, V(x), HIDDEN, 1, V(nw1), eps, V(q))
            L.rt_gemm_residual_dev(R, V(o), HIDDEN, HIDDEN, V(xa), HIDDEN, 1, V(x), V(x))
            L.rt_gemv_swiglu_norm_dev(R, V(g), V(u), FFN, HIDDEN, V(x), HIDDEN, 1, V(nw2), eps, V(h))
            L.rt_gemm_residual_dev(R, V(d), HIDDEN, FFN, V(h), FFN, 1, V(x), V(x))

    per = LAYERS * (alg_bytes(QKV, HIDDEN, 1) + alg_bytes(HIDDEN, HIDDEN, 1) + alg_bytes(FFN, HIDDEN, 1, pair=True) + alg_bytes(HIDDEN, FFN, 1))
    out = {"bytes_32_layers": per}
    for key, fn, apart in (("products_only", bare, False), ("epilogues_fused", with_epilogues, False), ("epilogues_apart", with_epilogues, True)):
        old = b.rt.set_epi_apart(apart)
        try:
            fn()
            b.rt.sync()
            L.rt_graph_begin(R)
            fn()
            g = L.rt_graph_end(R)
            L.rt_graph_launch(R, c.c_void_p(g))
            ms = b.timed(lambda: L.rt_graph_launch(R, c.c_void_p(g)), 20)
            L.rt_graph_free(R, c.c_void_p(g))
        finally:
            b.rt.set_epi_apart(old)
        out[key] = {"us_per_32_layers": round(1e3 * ms, 2), "GB/s": round(per / ms / 1e6, 1)}
    out["fused_saves_us_per_layer"] = round((out["epilogues_apart"]["us_per_32_layers"] - out["epilogues_fused"]["us_per_32_layers"]) / LAYERS, 3)
    for Lw in layers:
        for w in Lw:
            b.rt.free(w)
    for p in (x, xa, nw1, nw2, q, h, y):
        b.rt.free(p)
    return out


def gguf_load(b):
    """The GGUF load path: a file holding one 9B layer's five Q8_0 matrices (QKV 6144x4096, out
    4096x4096, gate and up 12288x4096, down 4096x12288: 205 MB) read by rt_gguf_read and uploaded by
    rt_gguf_upload (pread into pinned chunks, copy, repack to form S on the GPU), from the page
    cache. The reference repacks the same bytes in place on its CPU team instead (engine.c:303-316)."""
    import shutil
    import tempfile

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_file as gf

    F, H, Q = 12288, HIDDEN, 6144
    shapes = [("blk.0.attn_qkv.weight", Q, H), ("blk.0.attn_output.weight", H, H), ("blk.0.ffn_gate.weight", F, H),
              ("blk.0.ffn_up.weight", F, H), ("blk.0.ffn_down.weight", H, F)]
    rng = np.random.default_rng(5)
    tensors = [{"name": n, "dims": [k, r], "type": gf.Q8_0, "data": rng.integers(0, 256, r * k // 32 * 34, dtype=np.uint8).tobytes()}
               for n, r, k in shapes]
    d = tempfile.mkdtemp(prefix="q8gguf")
    try:
        path = os.path.join(d, "layer.gguf")
        gf.write(path, [("general.architecture", gf.STR, "qwen35")], tensors)
        times = []
        for _ in range(5):
            t0 = time.perf_counter()
            g = b.q8rt.GGUF(path)
            g.upload(b.rt)
            times.append(time.perf_counter() - t0)
            nbytes = g.h.q8_bytes
            g.close()
        s = statistics.median(times)
        return {"bytes": nbytes, "ms": round(s * 1e3, 2), "GB/s": round(nbytes / s / 1e9, 2), "runs": len(times)}
    finally:
        shutil.rmtree(d, ignore_errors=True)


def layers_2b(b):
    """Config 2: 24 layers of QKV 3072x2048, out 2048x2048, gate/up 6144x2048 (fused), down 2048x6144,
    one graph; beside it its floor, a graph of the same 96 positions as pure reads of each product's
    bytes on its own grid (rt_q8_read_dev), as for the 9B token."""
    H, F, Q = 2048, 6144, 2048 + 2 * 512
    layers = [(b.matrix(Q, H), b.matrix(H, H), b.matrix(F, H), b.matrix(F, H), b.matrix(H, F)) for _ in range(24)]
    xh, h, yq, yo, yd = b.vec(H), b.vec(F), b.vec(Q), b.vec(H), b.vec(H)
    sink = b.vec(F)  # a word a workgroup: fewer workgroups than the largest product's rows
    V = c.c_void_p

    def run():
        for qkv, o, g, u, d in layers:
            b.gemm(qkv, Q, H, xh, 1, yq)
            b.gemm(o, H, H, xh, 1, yo)
            b.pair(g, u, F, H, xh, 1, h)
            b.gemm(d, H, F, h, 1, yd)

    def floor():
        for qkv, o, g, u, d in layers:
            b.lib.rt_q8_read_dev(b.R, V(qkv), None, Q, H, V(xh), H, 1, V(sink))
            b.lib.rt_q8_read_dev(b.R, V(o), None, H, H, V(xh), H, 1, V(sink))
            b.lib.rt_q8_read_dev(b.R, V(g), V(u), F, H, V(xh), H, 1, V(sink))
            b.lib.rt_q8_read_dev(b.R, V(d), None, H, F, V(h), F, 1, V(sink))

    per = 24 * (alg_bytes(Q, H, 1) + alg_bytes(H, H, 1) + alg_bytes(F, H, 1, pair=True) + alg_bytes(H, F, 1))
    out = {}
    for key, fn in (("", run), ("floor_", floor)):
        b.lib.rt_graph_begin(b.R)
        fn()
        g = b.lib.rt_graph_end(b.R)
        b.lib.rt_graph_launch(b.R, V(g))
        ms = b.timed(lambda: b.lib.rt_graph_launch(b.R, V(g)), 20)
        b.lib.rt_graph_free(b.R, V(g))
        out[f"{key}us_per_pass"] = round(1e3 * ms, 2)
        out[f"{key}GB/s"] = round(per / ms / 1e6, 1)
    for L in layers:
        for w in L:
            b.rt.free(w)
    out["bytes"] = per
    return out


def cpu_baseline(b, layer, seconds):
    """The reference's host path on this host's cores over one 9B layer's products (bounded sample),
    and, beside it, the same path on configs 1, 4 (M = 16) and 5 (M = 4), a few seconds each."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    threads = min(16, len(os.sched_getaffinity(0)))
    shapes = [("qkv", QKV, HIDDEN), ("out", HIDDEN, HIDDEN), ("gate", FFN, HIDDEN), ("up", FFN, HIDDEN), ("down", HIDDEN, FFN)]

    def host_rows(rows, cols, seed, dist=0, mu=0.0, sigma=0.02):
        """GGUF rows drawn on the GPU from their seed, copied to the host"""
        b.lib.rt_q8_fill_dev(b.R, c.c_void_p(b.staging), rows, cols, seed, dist, mu, sigma)
        raw = np.empty(q8_bytes(rows, cols), np.uint8)
        b.rt.from_dev(raw, b.staging)
        return raw

    seed0 = layer["seed0"]
    mats = [(rows, cols, host_rows(rows, cols, seed0 + i)) for i, (name, rows, cols) in enumerate(shapes)]
    rng = np.random.default_rng(0)
    nbytes = sum(alg_bytes(r, k, 1) for _, r, k in shapes)
    teams = []
    flags = "oracle"

    def reference_product(path):
        """the reference's team product from the build at path (oracle/_ref), its team made here"""
        from oracle_ffi import Reference

        ref = Reference(path)
        team = ref.lib.ref_team_create(threads)
        if not team:
            raise OSError("team")
        teams.append((ref, team))

        def product(form, rows, cols, x, t, y):
            if t == 1:
                ref.lib.ref_team_gemv_i(c.c_void_p(team), c.c_void_p(form.ctypes.data), rows, cols, c.c_void_p(x.ctypes.data), c.c_void_p(y.ctypes.data))
            else:
                ref.lib.ref_team_gemm_i(c.c_void_p(team), c.c_void_p(form.ctypes.data), rows, cols, c.c_void_p(x.ctypes.data), t,
                                        c.c_void_p(y.ctypes.data))
        return ref, product

    def done():
        for ref, team in teams:
            ref.lib.ref_team_destroy(c.c_void_p(team))

    try:
        # the value: the reference's code built with its own host flags; beside it, with -mfma
        ref, product = reference_product(os.path.join(ROOT, "oracle", "_ref", "libref_flags.so"))
        flags = "-O2 -ffp-contract=off (the reference's host flags, scripts/lib.sh:37)"
        kind = "reference"

        def prepare(rows, cols, raw):
            return ref.repack_i(raw, rows, cols)
    except (FileNotFoundError, OSError):
        from oracle_ffi import Oracle

        orc = Oracle()
        kind = "port"

        def prepare(rows, cols, raw):
            return raw

        def product(form, rows, cols, x, t, y):
            orc.lib.q8o_gemm_mt(c.c_void_p(form.ctypes.data), rows, cols, c.c_void_p(x.ctypes.data), cols, t, c.c_void_p(y.ctypes.data), threads)
        done = lambda: None  # noqa: E731

    def median_time(run, budget, at_least=3, at_most=200):
        run()  # warm-up, dropped (src/bench/gemv_bench.c:113-125)
        times = []
        t_end = time.perf_counter() + budget
        while len(times) < at_least or (time.perf_counter() < t_end and len(times) < at_most):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        return statistics.median(times), len(times)

    def job(rows, cols, raw, t):
        x = rng.standard_normal((t, cols), dtype=np.float32)
        return (prepare(rows, cols, raw), rows, cols, x, t, np.empty((t, rows), np.float32))

    try:
        layer_jobs = [job(rows, cols, raw, 1) for rows, cols, raw in mats]
        med, n = median_time(lambda: [product(*j) for j in layer_jobs], seconds)
        out = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind, "flags": flags,
               "sample": f"one 9B decode layer (QKV 6144x4096, out 4096x4096, gate and up 12288x4096, down 4096x12288: {nbytes} B), "
                         f"median of {n} passes after one warm-up, {threads} threads pinned to this host's CPUs",
               "ms_per_layer": round(1e3 * med, 2), "host_cpus": os.cpu_count()}
        configs = {}
        # config 1: the 4096x4096 GEMV (seed 0 rows, as the parity fixtures)
        j1 = job(HIDDEN, HIDDEN, host_rows(HIDDEN, HIDDEN, 0), 1)
        med, n = median_time(lambda: product(*j1), 2.0)
        configs["gemv_4096x4096"] = {"ms": round(1e3 * med, 3), "GB/s": round(alg_bytes(HIDDEN, HIDDEN, 1) / med / 1e9, 3), "passes": n}
        # config 4: the prompt GEMM, M = 16, gate/up shape
        j4 = job(FFN, HIDDEN, host_rows(FFN, HIDDEN, 7), 16)
        med, n = median_time(lambda: product(*j4), 4.0, at_least=2)
        configs["gemm_m16_12288x4096"] = {"ms": round(1e3 * med, 2), "GFLOPS": round(2.0 * 16 * FFN * HIDDEN / med / 1e9, 2), "passes": n}
        # config 5: verify at M = 4, gate and up then down, heavy-tailed scales
        kw = dict(dist=1, mu=float(np.log(0.002)), sigma=1.0)
        j5 = [job(FFN, HIDDEN, host_rows(FFN, HIDDEN, 8, **kw), 4), job(FFN, HIDDEN, host_rows(FFN, HIDDEN, 9, **kw), 4),
              job(HIDDEN, FFN, host_rows(HIDDEN, FFN, 10, **kw), 4)]
        med, n = median_time(lambda: [product(*j) for j in j5], 4.0, at_least=2)
        v_bytes = alg_bytes(FFN, HIDDEN, 4, pair=True) + alg_bytes(HIDDEN, FFN, 4)
        configs["verify_m4_gate_up_down"] = {"ms": round(1e3 * med, 2), "GB/s": round(v_bytes / med / 1e9, 3), "passes": n}
        out["configs"] = configs
        if kind == "reference":
            # the same layer on the build with -mfma, its team made once the first one is gone (a
            # team pins its calling thread; destroying it gives the thread its CPUs back)
            done()
            teams.clear()
            try:
                _, mfma_product = reference_product(os.path.join(ROOT, "oracle", "_ref", "libref.so"))
                med2, n2 = median_time(lambda: [mfma_product(*j) for j in layer_jobs], seconds / 2)
                out["variants"] = {"-mfma": {"value": round(nbytes / med2 / 1e9, 3), "unit": "GB/s", "ms_per_layer": round(1e3 * med2, 2),
                                             "passes": n2, "flags": "-O2 -ffp-contract=off -mfma (fmaf inlined; the same bits)"}}
            except (FileNotFoundError, OSError) as e:
                out["variants"] = {"-mfma": {"error": f"not timed: {e}"}}
    finally:
        done()
    return out


CALIB_BYTES = 1 << 30
PROFILES = os.path.join(ROOT, "profiles")
DECODE_PROFILE = os.path.join(PROFILES, "gemv_decode_9b_m1.md")
PROFILE_CMDS = [
    "rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_stats -o run -- python3 bench.py --steps 20 --warmup 3 "
    "--no-cpu --no-extra --calib > gpurun_out/prof_stats.log 2>&1",
    "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/prof_fetch -o run -- python3 bench.py --steps 2 --warmup 1 --no-cpu "
    "--no-extra --calib",
    "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/prof_write -o run -- python3 bench.py --steps 2 --warmup 1 --no-cpu "
    "--no-extra --calib",
    "python3 bench.py --summarize gpurun_out",
]


def _kname(full):
    """rocprof's kernel name without the return type and the argument list."""
    n = full.split("(")[0].strip()
    return n[5:] if n.startswith("void ") else n


BUILD = os.path.join(ROOT, "intel-phi-apl_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"


def kernel_registers(objs=("q8_kernels.o", "q8_gemm.o"), arch="gfx950"):
    """{kernel name as rocprof prints it: (VGPRs, AGPRs, SGPRs, scratch bytes a lane)} from the metadata
    of the gfx950 code objects in the library's own build (each object's offload bundle unbundled),
    or {} where the build or the tools are missing. rocprof's kernel trace reports a VGPR count of
    its own that is half the code object's for these kernels, so the profiles take these."""
    import re
    import tempfile

    regs = {}
    with tempfile.TemporaryDirectory() as d:
        for obj in objs:
            fb, co = os.path.join(d, obj + ".fatbin"), os.path.join(d, obj + ".co")
            try:
                subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", os.path.join(BUILD, obj), fb], check=True, capture_output=True)
                subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o", f"--input={fb}",
                                f"--targets=hipv4-amdgcn-amd-amdhsa--{arch}", f"--output={co}"], check=True, capture_output=True)
                notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", co], check=True, capture_output=True, text=True).stdout
            except (OSError, subprocess.CalledProcessError):
                continue
            found = []
            for block in re.split(r"\n  - \.agpr_count", notes)[1:]:
                field = lambda k: re.search(rf"\.{k}:\s+(\S+)", block)  # noqa: E731
                if not field("name"):
                    continue
                found.append((field("name").group(1), (int(field("vgpr_count").group(1)), int(re.match(r":\s+(\d+)", block).group(1)),
                                                        int(field("sgpr_count").group(1)), int(field("private_segment_fixed_size").group(1)))))
            try:
                names = subprocess.run(["c++filt"], input="\n".join(n for n, _ in found), check=True, capture_output=True, text=True).stdout.split("\n")
            except (OSError, subprocess.CalledProcessError):
                continue
            for (_, r), dn in zip(found, names):
                regs[_kname(dn)] = r
    return regs


def waves_by_registers(vgprs, agprs):
    """Waves a SIMD the register file allows (512 a lane, VGPRs and AGPRs each in blocks of 8), at most 8."""
    used = -(-vgprs // 8) * 8 + -(-agprs // 8) * 8
    return min(8, 512 // used) if used else 8


LDS_BYTES = 160 * 1024


def occupancy_cells(regs, name, lds, wg_threads):
    """'VGPRs | waves a SIMD at most, by registers / by LDS' for a kernel (its registers from the code
    object, its LDS a workgroup and workgroup size from the kernel trace)."""
    r = regs.get(name)
    if not r:
        return "? | ?"
    waves_wg = max(1, wg_threads // 64)
    by_lds = (LDS_BYTES // lds) * waves_wg / 4 if lds else 8
    return f"{r[0]} | {waves_by_registers(r[0], r[1])} / {min(8, by_lds):g}"


def summarize(run_dir, out=DECODE_PROFILE):
    """profiles/gemv_decode_9b_m1.md from the three rocprofv3 runs of PROFILE_CMDS: per product of the
    token, the kernel, its average duration in the kernel trace and in the benchmark's own events,
    and its HBM bytes per launch from FETCH_SIZE and WRITE_SIZE, each scaled by what the counter
    reads for the plain copy kernel over CALIB_BYTES."""
    import csv
    from collections import defaultdict

    line = next(json.loads(l) for l in open(os.path.join(run_dir, "prof_stats.log")) if l.startswith('{"metric"'))
    trace = defaultdict(list)
    for r in csv.DictReader(open(os.path.join(run_dir, "prof_stats", "run_kernel_trace.csv"))):
        g = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        trace[(_kname(r["Kernel_Name"]), g)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    counters = {}
    for cname, sub in (("FETCH_SIZE", "prof_fetch"), ("WRITE_SIZE", "prof_write")):
        acc = defaultdict(list)
        for r in csv.DictReader(open(os.path.join(run_dir, sub, "run_counter_collection.csv"))):
            if r["Counter_Name"] == cname:
                acc[(_kname(r["Kernel_Name"]), int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
        counters[cname] = {k: statistics.fmean(v) for k, v in acc.items()}
    ck = ("copy16", CALIB_BYTES // 16)
    scale = {n: CALIB_BYTES / (counters[n][ck] * 1024.0) for n in counters}
    stats = list(csv.DictReader(open(os.path.join(run_dir, "prof_stats", "run_kernel_stats.csv"))))
    rows, traffic = [], {}
    for shape, k in line["kernels_9b"].items():
        key = (k["kernel"], k["grid"])
        tr = trace.get(key, [])
        f, w = counters["FETCH_SIZE"].get(key), counters["WRITE_SIZE"].get(key)
        tb = None if f is None or w is None else round(1024.0 * (f * scale["FETCH_SIZE"] + w * scale["WRITE_SIZE"]))
        traffic[f"{k['kernel']} grid {k['grid']}"] = {"shape": shape, "traffic": tb, "alg_bytes": k["alg_bytes"],
                                                       "trace_us": round(statistics.fmean(tr), 3) if tr else None}
        rows.append(f"| {shape} | `{k['kernel']}` | {k['grid']} | {len(tr)} | {statistics.fmean(tr) if tr else float('nan'):.2f} | {k['us']:.2f} | "
                    f"{f if f is not None else float('nan'):.1f} | {w if w is not None else float('nan'):.1f} | {tb} | {k['alg_bytes']} | "
                    f"{(tb / k['alg_bytes']) if tb else float('nan'):.4f} |")
    roof = line["roofline"]
    text = [f"# Decode GEMV kernels, 9B-class token at M = 1 (rocprofv3)", "",
            f"Device: {line['device']}. Workload: {line['config']['workload']}.", "",
            "Commands (from the repository root; each rocprofv3 run on its own):", "", "```"] + PROFILE_CMDS + ["```", "",
            f"Token under the kernel trace: {line['ms_per_step']} ms with the graph, {line['eager_ms_per_step']} ms eager (the trace "
            "slows graph replays; the unprofiled figures are the benchmark's).", "",
            "## Kernel statistics (kernel trace, all launches of the run)", "",
            "| Kernel | Calls | Average ns | Min ns | Max ns | % of time |", "|---|---|---|---|---|---|"]
    for r in stats:
        text.append(f"| `{_kname(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']):.1f} | {r['MinNs']} | {r['MaxNs']} | {r['Percentage']} |")
    text += ["", "## Per product of the token", "",
             f"Counter yardstick: the copy kernel over {CALIB_BYTES} B reads FETCH_SIZE "
             f"{counters['FETCH_SIZE'][ck]:.1f} KiB and WRITE_SIZE {counters['WRITE_SIZE'][ck]:.1f} KiB per launch, so "
             f"FETCH_SIZE is scaled by {scale['FETCH_SIZE']:.4f} and WRITE_SIZE by {scale['WRITE_SIZE']:.4f}.", "",
             "| Product | Kernel | Grid (threads) | Launches traced | Trace avg us | Bench event avg us (under the trace) | FETCH_SIZE KiB | WRITE_SIZE KiB | "
             "HBM bytes (scaled) | Algorithmic bytes | HBM / algorithmic |", "|---|---|---|---|---|---|---|---|---|---|---|"] + rows
    dk = roof["kernel"].split(" (")[0] + " grid " + roof["kernel"].rsplit("grid ", 1)[1].rstrip(")")
    dt = traffic.get(dk, {})
    if dt.get("trace_us"):
        text += ["", f"Dominant kernel: {roof['kernel']}: {dt['trace_us']} us per launch in the kernel trace, so "
                 f"{roof['bytes_per_launch'] / dt['trace_us'] / 1e3:.1f} GB/s algorithmic = "
                 f"{100 * roof['bytes_per_launch'] / dt['trace_us'] / 1e3 / HBM_PEAK_GBS:.1f} % of {HBM_PEAK_GBS:.0f} GB/s (the unprofiled "
                 "benchmark's events time the same launches; the tracer leaves the GPU idle between dispatches — this run's token took "
                 f"{line['ms_per_step']} ms with the graph — and a kernel's traced duration runs above what the untraced events measure, the more so the shorter the kernel, so "
                 "this fraction is the conservative one)."]
    text += ["",
             "Machine-readable (read by bench.py for roofline.traffic):", "", "```json", json.dumps(traffic), "```", ""]
    os.makedirs(os.path.dirname(out), exist_ok=True)
    open(out, "w").write("\n".join(text))
    print(f"wrote {out}")


GEMM_PROFILE = os.path.join(PROFILES, "gemm_prompt_9b_ffn.md")
GEMM_PROFILE_CMDS = [
    "rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/gprof_stats -o run -- python3 bench.py --only prompt_gemm "
    "> gpurun_out/gprof_stats.log 2>&1",
    "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/gprof_fetch -o run -- python3 bench.py --only prompt_gemm",
    "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_INSTS_MFMA GRBM_GUI_ACTIVE --output-format csv "
    "-d gpurun_out/gprof_mfma -o run -- python3 bench.py --only prompt_gemm",
    "rocprofv3 --pmc SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_INST_ANY SQ_INSTS_VMEM_RD SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS "
    "GRBM_GUI_ACTIVE --output-format csv -d gpurun_out/gprof_sq -o run -- python3 bench.py --only prompt_gemm,draft_head "
    "> gpurun_out/gprof_sq.log 2>&1",
    "rocprofv3 --pmc TA_TA_BUSY_sum TA_ADDR_STALLED_BY_TC_CYCLES_sum TD_TD_BUSY_sum TD_TC_STALL_sum TCP_TCP_TA_DATA_STALL_CYCLES_sum "
    "TCP_PENDING_STALL_CYCLES_sum TCP_TCC_READ_REQ_LATENCY_sum TCP_TCC_READ_REQ_sum GRBM_GUI_ACTIVE --output-format csv "
    "-d gpurun_out/gprof_ta -o run -- python3 bench.py --only prompt_gemm,draft_head",
    "python3 bench.py --summarize-gemm gpurun_out",
]
GEMM_STALL_COUNTERS = ("SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_INST_ANY", "SQ_INSTS_VMEM_RD", "SQ_INSTS_VALU",
                       "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "TA_TA_BUSY_sum", "TA_ADDR_STALLED_BY_TC_CYCLES_sum", "TD_TD_BUSY_sum",
                       "TD_TC_STALL_sum", "TCP_TCP_TA_DATA_STALL_CYCLES_sum", "TCP_PENDING_STALL_CYCLES_sum", "TCP_TCC_READ_REQ_LATENCY_sum",
                       "TCP_TCC_READ_REQ_sum")


def summarize_gemm(run_dir, out=GEMM_PROFILE, xcds=8, simds=1024):
    """profiles/gemm_prompt_9b_ffn.md from the three rocprofv3 runs of GEMM_PROFILE_CMDS: per GEMM
    kernel and grid, its mean duration (kernel trace), HBM bytes (FETCH_SIZE, scaled as for the
    decode profile: x2.0), and MFMA utilisation = SQ_VALU_MFMA_BUSY_CYCLES over (GRBM_GUI_ACTIVE per
    XCD x SIMDs), with the bf16 MFMA ops the counters saw (512 flop a MOP) against the issued work."""
    import csv
    from collections import defaultdict

    line = json.loads(next(l for l in open(os.path.join(run_dir, "gprof_stats.log")) if l.startswith('{"prompt_gemm"')))["prompt_gemm"]
    trace, wg_shape = defaultdict(list), {}
    for r in csv.DictReader(open(os.path.join(run_dir, "gprof_stats", "run_kernel_trace.csv"))):
        g = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        trace[(_kname(r["Kernel_Name"]), g)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        wg_shape[(_kname(r["Kernel_Name"]), g)] = (int(r.get("LDS_Block_Size") or 0), int(r.get("Workgroup_Size_X") or 64))
    regs = kernel_registers()
    cnt = defaultdict(lambda: defaultdict(list))
    stall = defaultdict(lambda: defaultdict(list))  # the two stall passes, each with its own GRBM_GUI_ACTIVE
    for sub in ("gprof_fetch", "gprof_mfma", "gprof_sq", "gprof_ta"):
        path = os.path.join(run_dir, sub, "run_counter_collection.csv")
        if sub in ("gprof_sq", "gprof_ta") and not os.path.exists(path):
            continue
        for r in csv.DictReader(open(path)):
            key = (_kname(r["Kernel_Name"]), int(r["Grid_Size"]))
            if sub in ("gprof_sq", "gprof_ta"):
                stall[key][(sub, r["Counter_Name"])].append(float(r["Counter_Value"]))
            else:
                cnt[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
    mean = lambda v: statistics.fmean(v) if v else float("nan")  # noqa: E731
    rows = []
    for shape, k in line.items():
        m = int(shape.split()[0][1:])
        r_, c_ = (int(v) for v in shape.split()[1].split("x"))
        name = k["kernel"]
        # rocprof reports the grid as x*y*z threads, as the bench line does: match on name and grid
        key = (name, k["grid"])
        c = cnt.get(key, {})
        busy, gui = mean(c.get("SQ_VALU_MFMA_BUSY_CYCLES", [])), mean(c.get("GRBM_GUI_ACTIVE", []))
        mops = mean(c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", []))
        util = busy / (gui / xcds * simds) if gui == gui and gui > 0 else float("nan")
        mg = 1 if name.startswith("gemm_xres") else int(name.split("<")[1].split(",")[0])  # gemm_xres: one token tile
        issued = 2.0 * 3 * (16 * mg * -(-(-(-m // 16)) // mg)) * r_ * c_  # the token tiles the kernel runs: whole groups of MG
        tr = trace.get(key, [])
        # the floor (M <= 16): read_xres on the x-resident kernel's grid, from the trace and the bench line
        fl, ftr = k.get("floor_us"), trace.get((name.replace("gemm_xres", "read_xres"), k["grid"]), [])
        floor = "—" if fl is None else f"{mean(ftr):.2f} / {fl:.2f}" if ftr else f"— / {fl:.2f}"
        rows.append(f"| {shape} | `{name}` | {mean(tr):.2f} | {k['kernel_us']:.2f} | {k['product_us']:.2f} | {floor} | {k['GFLOPS']:.0f} | "
                    f"{2.0 * mean(c.get('FETCH_SIZE', [])) * 1024 / 1e6:.1f} | {alg_bytes(r_, c_, m) / 1e6:.1f} | {100 * util:.1f} | "
                    f"{mops * 512 / issued:.3f} | {occupancy_cells(regs, name, *wg_shape.get(key, (0, 64)))} |")
    text = ["# Prompt / verify GEMM on the matrix cores, 9B FFN shapes (rocprofv3)", "",
            "Workload: Y = X W^T, X F32 [M x cols], W Q8_0 gate/up 12288x4096 and down 4096x12288, M = 16, 40, 64; each product over "
            ">= 512 MB of rotated weight copies. The contraction runs as bf16 MFMA on three exact limbs of x (3x the flops of the "
            "product, tokens padded to 16).", "",
            "Commands (from the repository root; each rocprofv3 run on its own):", "", "```"] + GEMM_PROFILE_CMDS + ["```", "",
            "| Product | Kernel | Trace avg us | Bench kernel us | Bench product us (with the partial sum) | Floor us (trace / bench) | "
            "GFLOP/s (product) | HBM MB (FETCH_SIZE x2) | Algorithmic MB | MFMA busy % | counted bf16 MFMA flop / issued | VGPRs a lane | "
            "Waves a SIMD at most (registers / LDS) |", "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    text += rows
    text += ["", f"MFMA busy % = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {xcds} XCDs x {simds} SIMDs). Counted flop = "
             "SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512; issued = 2 x 3 limbs x the token tiles the kernel runs (whole groups of MG "
             "tiles of 16: at M = 40, 4 tiles, one of them all padding) x rows x cols. Counters are per (kernel, grid): "
             "products that launch the same kernel on the same grid share one average. VGPRs a lane from the library's gfx950 "
             "code object; the waves a SIMD they allow (512 registers a lane) and those the workgroup's LDS allows (160 KiB a CU, "
             "the LDS from the kernel trace), at most 8. Floor (M = 16): `read_xres`, the x-resident kernel's own loads (x, scales, "
             "weights through the same two register sets) on its grid with no arithmetic (rt_q8_read_dev at 16 tokens).", ""]
    if stall:
        dh = None
        for l in open(os.path.join(run_dir, "gprof_sq.log")) if os.path.exists(os.path.join(run_dir, "gprof_sq.log")) else []:
            if l.startswith('{"draft_head"'):
                dh = json.loads(l)["draft_head"]
        keyed = [(shape, (k["kernel"], k["grid"])) for shape, k in line.items()]
        if dh and "kernel" in dh:
            keyed.append((f"decode draft head {DRAFT}x{HIDDEN}, M=1 (contrast)", (dh["kernel"], dh["grid"])))
        text += ["## Where the waves wait (two more counter passes)", "",
                 f"Per kernel and grid, the kernel's cycles K = GRBM_GUI_ACTIVE / {xcds} of the same pass; a CU's TA, TD and TCP "
                 f"count each on their own (256 of each; their _sum over the device / (256 x K) is the share of a unit's cycles); "
                 f"SQ_WAVE_CYCLES and SQ_WAIT_INST_ANY are in quad-cycles (x 4). VALU busy % is an estimate from instruction "
                 f"counts: (SQ_INSTS_VALU - SQ_INSTS_MFMA) x 4 cycles (a wave64 instruction on a 16-lane SIMD) over K x {simds} "
                 "SIMDs. The draft head's decode kernel (1 KiB of one row a load instruction, every load of a wave issued at "
                 "once) streams at 78 % of HBM: the contrast.", "",
                 "| Product | Kernel | Waves a SIMD | Wave cycles waiting % | VALU busy % (est.) | TA busy % | TA stalled by TCP % | "
                 "TD stalled by TCP % | TCP stalled on TA data % | TCP pending % | L2 read latency cycles | Loads a wave | "
                 "VALU instructions a wave | MFMA instructions a wave | LDS instructions a wave |",
                 "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
        for shape, key in keyed:
            st = stall.get(key, {})
            g = lambda sub, n: mean(st.get((sub, n), []))  # noqa: E731
            ksq, kta = g("gprof_sq", "GRBM_GUI_ACTIVE") / xcds, g("gprof_ta", "GRBM_GUI_ACTIVE") / xcds
            cu = 256.0
            waves = g("gprof_sq", "SQ_WAVES")
            text.append(f"| {shape} | `{key[0]}` | {4 * g('gprof_sq', 'SQ_WAVE_CYCLES') / (ksq * simds):.2f} | "
                        f"{100 * g('gprof_sq', 'SQ_WAIT_INST_ANY') / g('gprof_sq', 'SQ_WAVE_CYCLES'):.1f} | "
                        f"{100 * 4 * (g('gprof_sq', 'SQ_INSTS_VALU') - g('gprof_sq', 'SQ_INSTS_MFMA')) / (ksq * simds):.1f} | "
                        f"{100 * g('gprof_ta', 'TA_TA_BUSY_sum') / (cu * kta):.1f} | {100 * g('gprof_ta', 'TA_ADDR_STALLED_BY_TC_CYCLES_sum') / (cu * kta):.1f} | "
                        f"{100 * g('gprof_ta', 'TD_TC_STALL_sum') / (cu * kta):.1f} | {100 * g('gprof_ta', 'TCP_TCP_TA_DATA_STALL_CYCLES_sum') / (cu * kta):.1f} | "
                        f"{100 * g('gprof_ta', 'TCP_PENDING_STALL_CYCLES_sum') / (cu * kta):.1f} | "
                        f"{g('gprof_ta', 'TCP_TCC_READ_REQ_LATENCY_sum') / g('gprof_ta', 'TCP_TCC_READ_REQ_sum'):.0f} | "
                        f"{g('gprof_sq', 'SQ_INSTS_VMEM_RD') / waves:.1f} | {g('gprof_sq', 'SQ_INSTS_VALU') / waves:.0f} | "
                        f"{g('gprof_sq', 'SQ_INSTS_MFMA') / waves:.0f} | {g('gprof_sq', 'SQ_INSTS_LDS') / waves:.0f} |")
        text.append("")
    open(out, "w").write("\n".join(text))
    print(f"wrote {out}")


VERIFY_PROFILE = os.path.join(PROFILES, "gemv_verify_9b_m2_m4.md")
VERIFY_PROFILE_CMDS = [
    "rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/vprof_stats -o run -- python3 bench.py --only verify "
    "> gpurun_out/vprof_stats.log 2>&1",
    "rocprofv3 --pmc FETCH_SIZE GRBM_GUI_ACTIVE --output-format csv -d gpurun_out/vprof_fetch -o run -- python3 bench.py --only verify",
    "rocprofv3 --pmc SQ_WAVE_CYCLES SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_WAIT_INST_ANY SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES "
    "SQ_INSTS_VMEM_RD SQ_INSTS_LDS GRBM_GUI_ACTIVE --output-format csv -d gpurun_out/vprof_sq -o run -- python3 bench.py --only verify",
    "python3 bench.py --summarize-verify gpurun_out",
]


def summarize_verify(run_dir, out=VERIFY_PROFILE, xcds=8, simds=1024):
    """profiles/gemv_verify_9b_m2_m4.md from the three rocprofv3 runs of VERIFY_PROFILE_CMDS: per verify
    kernel (the fused gate+up pair and down at M = 2, 3, 4), its mean duration (kernel trace), HBM
    bytes (FETCH_SIZE x2, as for the decode profile), VALU instructions a weight (MFMA ones
    included), the share of the SIMDs' cycles spent issuing VALU (SQ_INSTS_VALU x 4 cycles of a
    wave64 instruction over GRBM_GUI_ACTIVE / XCDs x SIMDs), MFMA instructions a weight and the
    share of the SIMDs' cycles their matrix cores are busy (SQ_VALU_MFMA_BUSY_CYCLES over the same),
    the waves resident a SIMD (SQ_WAVE_CYCLES, in quad-cycles, x 4 over the same) and the share of
    the waves' cycles spent waiting (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES)."""
    import csv
    from collections import defaultdict

    line = json.loads(next(l for l in open(os.path.join(run_dir, "vprof_stats.log")) if l.startswith('{"verify"')))["verify"]
    trace, wg_shape = defaultdict(list), {}
    for r in csv.DictReader(open(os.path.join(run_dir, "vprof_stats", "run_kernel_trace.csv"))):
        g = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        trace[(_kname(r["Kernel_Name"]), g)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        wg_shape[(_kname(r["Kernel_Name"]), g)] = (int(r.get("LDS_Block_Size") or 0), int(r.get("Workgroup_Size_X") or 64))
    regs = kernel_registers()
    cnt = defaultdict(lambda: defaultdict(list))
    for sub in ("vprof_fetch", "vprof_sq"):
        for r in csv.DictReader(open(os.path.join(run_dir, sub, "run_counter_collection.csv"))):
            cnt[(_kname(r["Kernel_Name"]), int(r["Grid_Size"]))][r["Counter_Name"]].append(float(r["Counter_Value"]))
    mean = lambda v: statistics.fmean(v) if v else float("nan")  # noqa: E731
    rows = []
    for m, res in line.items():
        t = int(m[1:])
        for what, k in res.items():
            pair = what == "fused_gate_up"
            r_, c_ = (FFN, HIDDEN) if pair else (HIDDEN, FFN)
            key = (k["kernel"], k["grid"])
            c = cnt.get(key, {})
            gui = mean(c.get("GRBM_GUI_ACTIVE", []))
            simd_cycles = gui / xcds * simds
            weights = (2 if pair else 1) * r_ * c_
            valu = mean(c.get("SQ_INSTS_VALU", []))
            mfma = mean(c.get("SQ_INSTS_MFMA", []))
            rows.append(f"| M={t} | {'gate+up pair' if pair else 'down'} {r_}x{c_} | `{k['kernel']}` | {mean(trace.get(key, [])):.2f} | {k['kernel_us']:.2f} | "
                        f"{100 * alg_bytes(r_, c_, t, pair) / k['kernel_us'] / 1e3 / HBM_PEAK_GBS:.1f} | {2.0 * mean(c.get('FETCH_SIZE', [])) * 1024 / 1e6:.1f} | "
                        f"{alg_bytes(r_, c_, t, pair) / 1e6:.1f} | {64 * valu / weights:.2f} | {100 * 4 * valu / simd_cycles:.1f} | "
                        f"{64 * mfma / weights:.3f} | {100 * mean(c.get('SQ_VALU_MFMA_BUSY_CYCLES', [])) / simd_cycles:.1f} | "
                        f"{4 * mean(c.get('SQ_WAVE_CYCLES', [])) / simd_cycles:.2f} | {100 * mean(c.get('SQ_WAIT_INST_ANY', [])) / mean(c.get('SQ_WAVE_CYCLES', [])):.1f} | "
                        f"{occupancy_cells(regs, k['kernel'], *wg_shape.get(key, (0, 64)))} |")
    text = ["# Speculative-verify products at 9B shapes, M = 2..4 tokens (rocprofv3)", "",
            "Workload: the fused gate+up pair SiLU(X Wg^T) * (X Wu^T), 2 x 12288x4096, then down 4096x12288, X F32 [M x cols], "
            "scales d = binary16(lognormal(ln 0.002, 1)), each product over >= 512 MB of rotated weight copies.", "",
            "Commands (from the repository root; each rocprofv3 run on its own):", "", "```"] + VERIFY_PROFILE_CMDS + ["```", "",
            "| M | Product | Kernel | Trace avg us | Bench kernel us | % of HBM peak | HBM MB (FETCH_SIZE x2) | Algorithmic MB | "
            "VALU instructions a weight (x64 lanes) | VALU issue % of SIMD cycles | MFMA instructions a weight (x64) | MFMA busy % of SIMD cycles | "
            "Waves a SIMD | Wave cycles waiting % | VGPRs a lane | Waves a SIMD at most (registers / LDS) |",
            "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    text += rows
    text += ["", f"VALU instructions a weight = SQ_INSTS_VALU x 64 lanes / weights (the pair counts both matrices; MFMA instructions are "
             "counted in it too). MFMA instructions a weight = SQ_INSTS_MFMA x 64 / weights (v_mfma_f32_4x4x1_16b_f32 takes 64 weights, 1.0); "
             "MFMA busy % = SQ_VALU_MFMA_BUSY_CYCLES over the SIMD cycles below. VALU issue % = "
             f"SQ_INSTS_VALU x 4 cycles (a wave64 instruction on a 16-lane SIMD) / (GRBM_GUI_ACTIVE / {xcds} XCDs x {simds} SIMDs). "
             "Waves a SIMD = SQ_WAVE_CYCLES (counted in quad-cycles, so x 4) over the same SIMD cycles; wave cycles waiting = "
             "SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (both in quad-cycles). Counters are per (kernel, grid). VGPRs a lane from the "
             "library's gfx950 code object (its metadata); the waves a SIMD they allow (512 registers a lane), and those the "
             "workgroup's LDS allows (160 KiB a CU, from the kernel trace), at most 8.", ""]
    open(out, "w").write("\n".join(text))
    print(f"wrote {out}")


def profiled_traffic(kname, grid, path=DECODE_PROFILE):
    """HBM bytes per launch of (kernel, grid) from the committed rocprofv3 summary, or None."""
    try:
        text = open(path).read()
        blob = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(blob).get(f"{kname} grid {grid}", {}).get("traffic")
    except (OSError, IndexError, ValueError):
        return None


def calib_copy(b):
    """Three copies of 1 GiB (4x the Infinity Cache) by the plain copy kernel: each reads and writes
    every byte once, so a --pmc run's FETCH_SIZE and WRITE_SIZE for it are the counters' yardstick."""
    src, dst = b.rt.alloc(CALIB_BYTES), b.rt.alloc(CALIB_BYTES)
    b.lib.rt_f32_fill_dev(b.R, c.c_void_p(src), CALIB_BYTES // 4, 99)
    ms = b.timed(lambda: b.lib.rt_dev_copy(b.R, c.c_void_p(dst), c.c_void_p(src), CALIB_BYTES), 3)
    log(f"calibration copy: {CALIB_BYTES} B read + written, {ms:.3f} ms, {2 * CALIB_BYTES / ms / 1e6:.1f} GB/s")
    b.rt.free(src)
    b.rt.free(dst)


def fresh_sections(keys):
    """Each section in a process of its own (this script with --only), run before this process
    touches the GPU: its buffers then land on fresh device memory, as the token's do. In one process,
    after other sections had allocated and freed their copies, the same kernels ran up to 15 %
    slower (the verify path at M = 2: 20.5 / 11.3 us alone, 21.9 / 12.4 with the token's 7.2 GB
    resident, 23.0 / 13.9 after freeing them)."""
    out = {}
    for key in keys:
        log(f"{key} ...")
        p = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", key], stdout=subprocess.PIPE, text=True, timeout=600)
        if p.returncode != 0:
            raise SystemExit(f"bench.py: section {key} failed (exit {p.returncode})")
        for line in p.stdout.splitlines():
            if line.startswith("{"):
                out.update(json.loads(line))
        log(f"  {json.dumps(out.get(key))}")
    return out


TRACE_PROFILE = os.path.join(PROFILES, "token_trace_9b_m1.md")
TRACE_PROFILE_CMDS = [
    "rocprofv3 --kernel-trace --output-format csv -d gpurun_out/ttrace -o run -- python3 bench.py --only token_trace "
    "> gpurun_out/ttrace.log 2>&1",
    "python3 bench.py --summarize-trace gpurun_out",
]


def _replays(rows, n, last_grid):
    """The trace's product kernels (rows: (name, grid, begin ns, end ns) in begin order) cut into
    tokens: a token ends with the output head (the kernel of grid last_grid, its last product); runs
    of any other length than n are dropped."""
    runs, cur = [], []
    for r in rows:
        cur.append(r)
        if r[1] == last_grid:
            runs.append(cur)
            cur = []
    return [r for r in runs if len(r) == n]


def summarize_trace(run_dir, out=TRACE_PROFILE):
    """profiles/token_trace_9b_m1.md from the kernel trace of `bench.py --only token_trace`: the graph
    replays and the eager tokens, each cut out of the trace by the idle stream around it; for the
    replay of median span, every kernel's begin (from the replay's first begin), duration and gap to
    the next kernel's begin; per product shape, the mean duration and gap over all replays."""
    import csv
    from collections import defaultdict

    line = next(json.loads(l) for l in open(os.path.join(run_dir, "ttrace.log")) if l.startswith('{"token_trace"'))["token_trace"]
    n = line["products"]
    rows = []
    for r in csv.DictReader(open(os.path.join(run_dir, "ttrace", "run_kernel_trace.csv"))):
        k = _kname(r["Kernel_Name"])
        if k.startswith(("gemv_", "gemm_", "read_k")):
            g = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            rows.append((k, g, int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    rows.sort(key=lambda r: r[2])
    runs = _replays(rows, n, VOCAB // 8 * 256)
    per = TRACE_REPLAYS + 1  # the untimed one first
    if len(runs) != 3 * per:
        raise SystemExit(f"summarize_trace: found {len(runs)} runs of {n} kernels, expected {3 * per}")
    text = ["# The 9B decode token kernel by kernel: one graph replay in the kernel trace (rocprofv3)", "",
            f"Workload: the 9B-class decode token at M = 1, {n} products ({LAYERS} x (QKV 6144x4096, out 4096x4096, gate+up 2x12288x4096 "
            f"fused, down 4096x12288) + head 151936x4096), {line['bytes_per_token']} B a token, recorded once as a HIP graph. "
            f"{TRACE_REPLAYS} replays, each alone on the stream (idle before and after), then {TRACE_REPLAYS} eager tokens the same way, "
            f"then {TRACE_REPLAYS} replays of the floor: a graph of the same 129 positions, each the product's loads on the product's grid "
            "and no arithmetic (rt_q8_read_dev); the first of each, untimed, is left out.", "",
            "Commands (from the repository root):", "", "```"] + TRACE_PROFILE_CMDS + ["```", "",
            f"Each replay's time on the stream's events in the same run (under the trace): graph median {line['graph']['ms_median']} ms "
            f"(min {line['graph']['ms_min']}), eager median {line['eager']['ms_median']} ms (min {line['eager']['ms_min']}), floor median "
            f"{line['floor']['ms_median']} ms (min {line['floor']['ms_min']}).", ""]

    def table(mode, group):
        spans = [(g[-1][3] - g[0][2]) / 1e3 for g in group]
        busy = [sum((r[3] - r[2]) / 1e3 for r in g) for g in group]
        gaps = [sum((g[i + 1][2] - g[i][3]) / 1e3 for i in range(len(g) - 1)) for g in group]
        med = sorted(range(len(group)), key=lambda i: spans[i])[len(group) // 2]
        text.extend([f"## {mode}", "",
                     f"Over the {len(group)} {mode} runs: span (first begin to last end) median {statistics.median(spans):.1f} us "
                     f"(min {min(spans):.1f}, max {max(spans):.1f}); kernels busy median {statistics.median(busy):.1f} us; gaps between "
                     f"kernels median {statistics.median(gaps):.1f} us in all, {statistics.median(gaps) / (n - 1):.3f} us a boundary.", ""])
        by = defaultdict(lambda: ([], []))
        for g in group:
            for i, r in enumerate(g):
                by[(r[0], r[1])][0].append((r[3] - r[2]) / 1e3)
                if i + 1 < len(g):
                    by[(r[0], r[1])][1].append((g[i + 1][2] - r[3]) / 1e3)
        text.extend(["Per kernel and grid, over every run:", "", "| Kernel | Grid (threads) | Launches | Mean duration us | Mean gap to the next us |",
                     "|---|---|---|---|---|"])
        for (k, gr), (d, gp) in sorted(by.items(), key=lambda kv: -sum(kv[1][0])):
            text.append(f"| `{k}` | {gr} | {len(d)} | {statistics.fmean(d):.3f} | {statistics.fmean(gp) if gp else float('nan'):.3f} |")
        g = group[med]
        t0 = g[0][2]
        text.extend(["", f"The {mode} run of median span ({spans[med]:.1f} us), kernel by kernel (us from its first begin):", "",
                     "| # | Kernel | Grid | Begin | End | Duration | Gap to the next |", "|---|---|---|---|---|---|---|"])
        for i, r in enumerate(g):
            gap = f"{(g[i + 1][2] - r[3]) / 1e3:.3f}" if i + 1 < len(g) else ""
            text.append(f"| {i} | `{r[0]}` | {r[1]} | {(r[2] - t0) / 1e3:.3f} | {(r[3] - t0) / 1e3:.3f} | {(r[3] - r[2]) / 1e3:.3f} | {gap} |")
        text.append("")

    table("graph", runs[1:per])
    table("eager", runs[per + 1:2 * per])
    table("floor", runs[2 * per + 1:])
    # product against floor, position class by position class (the layer's four products and the head)
    names = ["QKV 6144x4096", "out 4096x4096", "gate+up 2x12288x4096", "down 4096x12288"]
    text.extend(["## Product against its floor", "", "Mean over every graph replay and floor replay of the kernel durations at each position "
                 "of a layer (and the head): the product kernel, the pure read of the same bytes on the same grid, and the difference, "
                 "which is the product's own arithmetic and reductions past its loads.", "",
                 "| Position | Product us | Floor us | Product - floor us | Per token us |", "|---|---|---|---|---|"])
    tot = [0.0, 0.0]
    for j in range(5):
        idx = [n - 1] if j == 4 else [4 * l + j for l in range(LAYERS)]
        pd = statistics.fmean((g[i][3] - g[i][2]) / 1e3 for g in runs[1:per] for i in idx)
        fd = statistics.fmean((g[i][3] - g[i][2]) / 1e3 for g in runs[2 * per + 1:] for i in idx)
        tot[0] += pd * len(idx)
        tot[1] += fd * len(idx)
        text.append(f"| {names[j] if j < 4 else 'head 151936x4096'} | {pd:.3f} | {fd:.3f} | {pd - fd:.3f} | {(pd - fd) * len(idx):.1f} |")
    text.extend(["", f"Kernel time a token: products {tot[0]:.1f} us, floor {tot[1]:.1f} us, difference {tot[0] - tot[1]:.1f} us.", ""])
    os.makedirs(os.path.dirname(out), exist_ok=True)
    open(out, "w").write("\n".join(text))
    print(f"wrote {out}")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", metavar="SECTIONS", help="comma-separated sections to run instead of the full line (gemv_4096x4096, "
                    "draft_head, prompt_gemm, verify, 2b_layer_set, deltanet_round_9b, prompt_rounds_9b, host_pointers, gguf_load_9b_layer, "
                    "epilogues_9b); prints their results only")
    ap.add_argument("--summarize", metavar="DIR", help="write the rocprofv3 summary under profiles/ from DIR (the output of the "
                    "profile commands) and exit")
    ap.add_argument("--summarize-gemm", metavar="DIR", help="write the GEMM rocprofv3 summary under profiles/ from DIR and exit")
    ap.add_argument("--summarize-verify", metavar="DIR", help="write the verify-path rocprofv3 summary under profiles/ from DIR and exit")
    ap.add_argument("--summarize-trace", metavar="DIR", help="write the token-trace summary (a graph replay kernel by kernel) under "
                    "profiles/ from DIR and exit")
    ap.add_argument("--calib", action="store_true", help="also copy 1 GiB three times with the plain copy kernel (the yardstick "
                    "for the HBM byte counters of a rocprofv3 --pmc run)")
    a = ap.parse_args()
    if a.summarize:
        summarize(a.summarize)
        return
    if a.summarize_gemm:
        summarize_gemm(a.summarize_gemm)
        return
    if a.summarize_verify:
        summarize_verify(a.summarize_verify)
        return
    if a.summarize_trace:
        summarize_trace(a.summarize_trace)
        return
    if a.gpus != 1:
        print(f"bench.py: --gpus {a.gpus}: only one GPU is measured (every product runs on one MI355X; across GPUs the rows would "
              "shard by whole 16-row groups, each GPU computing its slice of y)", file=sys.stderr)
        sys.exit(2)
    sections = (("gemv_4096x4096", single_gemv), ("draft_head", draft_head), ("prompt_gemm", prompt_gemm), ("verify", verify_path),
                ("2b_layer_set", layers_2b), ("deltanet_round_9b", deltanet_round), ("prompt_rounds_9b", prompt_rounds),
                ("gguf_load_9b_layer", gguf_load), ("epilogues_9b", epilogues_9b))
    if a.only:
        sections = sections + (("token_trace", token_trace),)
        want = a.only.split(",")
        if "host_pointers" in want:  # the C harness, before this process touches the GPU
            print(json.dumps({"host_pointers": host_path()}), flush=True)
            want = [k for k in want if k != "host_pointers"]
            if not want:
                return
        q8rt = package()
        b = Bench(q8rt)
        for key, fn in sections:
            if key in want:
                print(json.dumps({key: fn(b)}), flush=True)
        b.rt.close()
        return
    extra = {}
    if not a.no_extra:
        extra = fresh_sections([key for key, _ in sections])
        log("host_pointers (the C harness) ...")
        extra["host_pointers"] = host_path()
        log(f"  {json.dumps(extra['host_pointers'])}")
    q8rt = package()
    b = Bench(q8rt)
    name, cus = b.rt.device_info()
    log(f"device: {name}, {cus} CUs")
    if a.calib:
        calib_copy(b)
    seed0 = b.seed + 1
    per_token, ms_graph, ms_eager, kernels, roof, layers = decode_9b(b, a.steps, a.warmup)
    layer0 = {"seed0": seed0}
    cpu = None
    if not a.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline(b, layer0, a.cpu_seconds)
        log(f"  {json.dumps(cpu)}")
    value = per_token / ms_graph / 1e6
    gm = extra.get("prompt_gemm", {}).get(f"M16 {FFN}x{HIDDEN}")
    line = {
        "metric": "Q8_0 GEMV HBM GB/s (% of peak) at 9B decode; M=16 GEMM GFLOPS",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "settle_replays": b.settle_replays,
        "ms_per_step": round(ms_graph, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (Q8_0 int8 weights, binary16 scales)",
        "data": "synthetic (seeded on the GPU: q uniform in [-127,127], d = binary16(|N(0,0.02)|/127), x ~ N(0,1))",
        "config": {"workload": "9B-class decode token, M=1: 32 x (QKV 6144x4096, out 4096x4096, gate+up 2x12288x4096 fused SiLU(g)*u, "
                               "down 4096x12288) + head 151936x4096; one HIP graph per token",
                   "bytes_per_token": per_token, "products_per_token": 4 * LAYERS + 1},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "eager_ms_per_step": round(ms_eager, 4),
        "floor_ms_per_step": round(b.floor_ms, 4),
        "floor_pct_of_hbm_peak": round(100 * per_token / b.floor_ms / 1e6 / HBM_PEAK_GBS, 2),
        "gemm_m16_gflops": gm["GFLOPS"] if gm else None,
        "gemm_m16_mfma_util": gm["mfma_util_kernel"] if gm else None,
        "roofline": roof,
        "cpu_baseline": cpu,
        "device": name,
        "kernels_9b": kernels,
        "configs": extra,
    }
    print(json.dumps(line), flush=True)
    b.rt.close()


if __name__ == "__main__":
    main()
