"""The benchmark's profile writers (bench.summarize, bench.summarize_gemm, bench.summarize_verify) on
small synthetic runs in rocprofv3's CSV layout: each product is matched to its own kernel and grid
(two products that share a kernel name on different grids stay apart), trace averages and counter
scaling come out as computed by hand, and the matrix-core table counts the x-resident kernel as one
token tile."""
import csv
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _csv(path, fields, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


def _trace(path, launches, wg=None):
    """launches: (kernel name, grid threads, [durations in us]); wg: {kernel name: (LDS bytes, workgroup threads)}"""
    rows, t = [], 1000
    for name, grid, durs in launches:
        lds, threads = (wg or {}).get(name, (0, 256))
        for d in durs:
            rows.append({"Kernel_Name": f"void {name}(unsigned char const*, long)", "Grid_Size_X": grid, "Grid_Size_Y": 1, "Grid_Size_Z": 1,
                         "Start_Timestamp": t, "End_Timestamp": t + int(round(d * 1000)), "LDS_Block_Size": lds, "Workgroup_Size_X": threads})
            t += 100000
    _csv(path, ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp", "End_Timestamp", "LDS_Block_Size", "Workgroup_Size_X"],
         rows)


def _counters(path, values):
    """values: (kernel name, grid, counter, [values])"""
    rows = [{"Kernel_Name": f"void {n}(float const*)", "Grid_Size": g, "Counter_Name": cn, "Counter_Value": v} for n, g, cn, vs in values for v in vs]
    _csv(path, ["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"], rows)


def test_decode_summary_matches_kernel_and_grid(tmp_path):
    run = tmp_path / "run"
    k = "gemv_k<1, 8, 1, 4, 0>"
    kernels_9b = {"gemv 4096x4096 t1": {"kernel": k, "grid": 131072, "us": 5.0, "alg_bytes": 17858560},
                  "gemv 6144x4096 t1": {"kernel": k, "grid": 196608, "us": 6.5, "alg_bytes": 26779648}}
    line = {"metric": "m", "kernels_9b": kernels_9b, "device": "gfx950", "config": {"workload": "w"}, "ms_per_step": 1.5,
            "eager_ms_per_step": 1.5,
            "roofline": {"kernel": f"{k} (gemv 6144x4096, t=1, grid 196608)", "bytes_per_launch": 26779648}}
    os.makedirs(run)
    (run / "prof_stats.log").write_text("noise\n" + json.dumps(line) + "\n")
    _trace(str(run / "prof_stats" / "run_kernel_trace.csv"), [(k, 131072, [5.0, 5.2]), (k, 196608, [7.0, 7.4, 7.2])])
    _csv(str(run / "prof_stats" / "run_kernel_stats.csv"), ["Name", "Calls", "AverageNs", "MinNs", "MaxNs", "Percentage"],
         [{"Name": f"void {k}(float const*)", "Calls": 5, "AverageNs": 6360.0, "MinNs": 5000, "MaxNs": 7400, "Percentage": 100.0}])
    ck = ("copy16", bench.CALIB_BYTES // 16)
    # the yardstick reads half its bytes on FETCH_SIZE and all on WRITE_SIZE: scales 2 and 1
    _counters(str(run / "prof_fetch" / "run_counter_collection.csv"),
              [(ck[0], ck[1], "FETCH_SIZE", [bench.CALIB_BYTES / 2048.0]), (k, 131072, "FETCH_SIZE", [8800.0, 8800.0]), (k, 196608, "FETCH_SIZE", [13100.0])])
    _counters(str(run / "prof_write" / "run_counter_collection.csv"),
              [(ck[0], ck[1], "WRITE_SIZE", [bench.CALIB_BYTES / 1024.0]), (k, 131072, "WRITE_SIZE", [16.0]), (k, 196608, "WRITE_SIZE", [24.0])])
    out = tmp_path / "decode.md"
    bench.summarize(str(run), out=str(out))
    text = out.read_text()
    blob = json.loads(text.split("```json", 1)[1].split("```", 1)[0])
    a, b = blob[f"{k} grid 131072"], blob[f"{k} grid 196608"]
    assert a["trace_us"] == pytest.approx(5.1) and b["trace_us"] == pytest.approx(7.2)
    assert a["traffic"] == round(1024 * (8800.0 * 2 + 16.0)) and b["traffic"] == round(1024 * (13100.0 * 2 + 24.0))
    assert "Dominant kernel" in text and "7.2 us per launch" in text


def test_gemm_summary_matches_grid_and_counts_the_x_resident_tile(tmp_path, monkeypatch):
    """Per (kernel, grid): trace mean, bench times, counted/issued MFMA work, and the occupancy cells:
    the code object's VGPRs (here stubbed) give 512 // 128 = 4 waves a SIMD, the x-resident
    workgroup's 113 KiB of LDS one workgroup a CU, 16 waves: 4 a SIMD; the streaming one's 76 KiB
    two, 8 a SIMD (at most 8)."""
    run = tmp_path / "run"
    xr, mf = "gemm_xres<2, 16, 8>", "gemm_mfma<3, 1, 2, 16>"
    monkeypatch.setattr(bench, "kernel_registers", lambda *a, **k: {xr: (128, 0, 54, 0), mf: (96, 0, 60, 0)})
    shapes = {"M16 12288x4096": (xr, 245760, 18.0, 12288, 4096, 16), "M16 4096x12288": (xr, 262144, 19.0, 4096, 12288, 16),
              "M40 12288x4096": (mf, 245760, 27.0, 12288, 4096, 40)}
    line = {"prompt_gemm": {s: {"kernel": n, "grid": g, "kernel_us": us, "product_us": us + 1, "GFLOPS": 1.0} for s, (n, g, us, _, _, _) in shapes.items()}}
    line["prompt_gemm"]["M16 12288x4096"]["floor_us"] = 14.5
    line["prompt_gemm"]["M16 4096x12288"]["floor_us"] = 15.25
    os.makedirs(run)
    (run / "gprof_stats.log").write_text(json.dumps(line) + "\n")
    rd = xr.replace("gemm_xres", "read_xres")  # the floor's kernel, on the same grid
    _trace(str(run / "gprof_stats" / "run_kernel_trace.csv"), [(xr, 245760, [17.0, 17.4]), (xr, 262144, [18.5]), (mf, 245760, [26.0, 28.0]),
                                                              (rd, 245760, [14.0, 14.2])], wg={xr: (115712, 1024), mf: (77824, 1024)})
    # issued bf16 MFMA flop = 2 x 3 limbs x the token tiles run x rows x cols; the counter counts 512 flop a MOP
    mops = {(n, g): 2.0 * 3 * (16 * (1 if n == xr else 3)) * r * c / 512 for n, g, _, r, c, _ in shapes.values()}
    _counters(str(run / "gprof_fetch" / "run_counter_collection.csv"), [(n, g, "FETCH_SIZE", [30000.0]) for (n, g) in mops])
    vals = []
    for (n, g), m in mops.items():
        vals += [(n, g, "SQ_INSTS_VALU_MFMA_MOPS_BF16", [m]), (n, g, "SQ_VALU_MFMA_BUSY_CYCLES", [1024.0]), (n, g, "GRBM_GUI_ACTIVE", [8.0 * 10])]
    _counters(str(run / "gprof_mfma" / "run_counter_collection.csv"), vals)
    out = tmp_path / "gemm.md"
    bench.summarize_gemm(str(run), out=str(out))
    rows = {l.split("|")[1].strip(): [c.strip() for c in l.split("|")[2:-1]] for l in out.read_text().splitlines() if l.startswith("| M")}
    assert rows["M16 12288x4096"][1] == "17.20" and rows["M16 4096x12288"][1] == "18.50" and rows["M40 12288x4096"][1] == "27.00"
    for s in shapes:
        assert rows[s][-3] == "1.000", s  # counted / issued: one token tile for gemm_xres, three for gemm_mfma<3, ...>
        assert rows[s][-4] == "10.0", s   # MFMA busy: 1024 cycles over (80 / 8 XCDs x 1024 SIMDs)
    assert rows["M16 12288x4096"][-2:] == ["128", "4 / 4"] and rows["M40 12288x4096"][-2:] == ["96", "5 / 8"]
    # the floor column: trace mean of read_xres on the product's grid / the bench's floor_us; none past M = 16
    assert rows["M16 12288x4096"][4] == "14.10 / 14.50" and rows["M16 4096x12288"][4] == "— / 15.25" and rows["M40 12288x4096"][4] == "—"


def test_gemm_stall_table_by_hand(tmp_path):
    """The GEMM profile's stall table, per kernel and grid, from the SQ pass and the TA/TD/TCP pass,
    each over its own GRBM_GUI_ACTIVE (summed over 8 XCDs): waves a SIMD and waiting from the
    quad-cycle counters, the VALU estimate from instruction counts (MFMAs left out, 4 cycles an
    instruction), the units' shares over 256 CUs, the L2 latency a request, counts a wave."""
    run = tmp_path / "run"
    xr = "gemm_xres<2, 16, 8>"
    line = {"prompt_gemm": {"M16 12288x4096": {"kernel": xr, "grid": 245760, "kernel_us": 18.0, "product_us": 19.0, "GFLOPS": 1.0}}}
    os.makedirs(run)
    (run / "gprof_stats.log").write_text(json.dumps(line) + "\n")
    _trace(str(run / "gprof_stats" / "run_kernel_trace.csv"), [(xr, 245760, [17.0])])
    _counters(str(run / "gprof_fetch" / "run_counter_collection.csv"), [(xr, 245760, "FETCH_SIZE", [30000.0])])
    _counters(str(run / "gprof_mfma" / "run_counter_collection.csv"), [(xr, 245760, "GRBM_GUI_ACTIVE", [80.0])])
    k = 1000.0  # the kernel's cycles
    sq = {"GRBM_GUI_ACTIVE": 8 * k, "SQ_WAVES": 3840.0, "SQ_WAVE_CYCLES": 1024 * k / 4 * 2.0, "SQ_WAIT_INST_ANY": 1024 * k / 4 * 2.0 * 0.3,
          "SQ_INSTS_VALU": 1024 * k / 4 * 0.4 + 500.0, "SQ_INSTS_MFMA": 500.0, "SQ_INSTS_LDS": 3840.0 * 7, "SQ_INSTS_VMEM_RD": 3840.0 * 27,
          "SQ_BUSY_CYCLES": 1.0}
    ta = {"GRBM_GUI_ACTIVE": 8 * k, "TA_TA_BUSY_sum": 256 * k * 0.32, "TA_ADDR_STALLED_BY_TC_CYCLES_sum": 256 * k * 0.22, "TD_TD_BUSY_sum": 1.0,
          "TD_TC_STALL_sum": 256 * k * 0.31, "TCP_TCP_TA_DATA_STALL_CYCLES_sum": 256 * k * 0.003, "TCP_PENDING_STALL_CYCLES_sum": 256 * k * 0.09,
          "TCP_TCC_READ_REQ_LATENCY_sum": 826.0 * 100, "TCP_TCC_READ_REQ_sum": 100.0}
    _counters(str(run / "gprof_sq" / "run_counter_collection.csv"), [(xr, 245760, n, [v]) for n, v in sq.items()])
    _counters(str(run / "gprof_ta" / "run_counter_collection.csv"), [(xr, 245760, n, [v]) for n, v in ta.items()])
    out = tmp_path / "gemm.md"
    bench.summarize_gemm(str(run), out=str(out))
    text = out.read_text().split("## Where the waves wait", 1)[1]
    row = [c.strip() for c in next(l for l in text.splitlines() if l.startswith("| M16")).split("|")[3:-1]]
    assert row == ["2.00", "30.0", "40.0", "32.0", "22.0", "31.0", "0.3", "9.0", "826", "27.0", "27", "0", "7"]


def test_verify_summary_per_kernel_and_grid(tmp_path):
    """bench.summarize_verify: each verify product (M, pair or down) is matched to its own kernel and
    grid; counters per weight and per SIMD cycle as computed by hand (GRBM_GUI_ACTIVE summed over 8
    XCDs, 1024 SIMDs, SQ_WAVE_CYCLES and SQ_WAIT_INST_ANY in quad-cycles)."""
    run = tmp_path / "run"
    F, H = bench.FFN, bench.HIDDEN
    pk, dk = "gemv_k<4, 8, 1, 4, 1>", "gemv_k<4, 16, 1, 12, 0>"
    line = {"verify": {"M4": {"fused_gate_up": {"kernel_us": 30.0, "kernel": pk, "grid": 196608},
                              "down": {"kernel_us": 20.0, "kernel": dk, "grid": 196608}}}}
    os.makedirs(run)
    (run / "vprof_stats.log").write_text("noise\n" + json.dumps(line) + "\n")
    _trace(str(run / "vprof_stats" / "run_kernel_trace.csv"), [(pk, 196608, [28.0, 28.4]), (dk, 196608, [16.5])])
    _counters(str(run / "vprof_fetch" / "run_counter_collection.csv"), [(pk, 196608, "FETCH_SIZE", [50000.0]), (dk, 196608, "FETCH_SIZE", [25000.0])])
    gui = 8.0 * 1000  # 1000 cycles a XCD: 1024000 SIMD cycles
    vals = []
    for k, w in ((pk, 2 * F * H), (dk, H * F)):
        vals += [(k, 196608, "SQ_INSTS_VALU", [w / 64 * 4.0]), (k, 196608, "SQ_INSTS_MFMA", [w / 64]), (k, 196608, "GRBM_GUI_ACTIVE", [gui]),
                 (k, 196608, "SQ_VALU_MFMA_BUSY_CYCLES", [102400.0]), (k, 196608, "SQ_WAVE_CYCLES", [512000.0]),
                 (k, 196608, "SQ_WAIT_INST_ANY", [128000.0])]
    _counters(str(run / "vprof_sq" / "run_counter_collection.csv"), vals)
    out = tmp_path / "verify.md"
    bench.summarize_verify(str(run), out=str(out))
    rows = [[c.strip() for c in l.split("|")[1:-1]] for l in out.read_text().splitlines() if l.startswith("| M=")]
    assert [r[1].split()[0] for r in rows] == ["gate+up", "down"]
    pair, down = rows
    assert pair[2] == f"`{pk}`" and pair[3] == "28.20" and down[3] == "16.50"
    assert pair[6] == f"{2.0 * 50000 * 1024 / 1e6:.1f}" and down[6] == f"{2.0 * 25000 * 1024 / 1e6:.1f}"  # FETCH_SIZE x2, KiB
    for r in rows:
        assert r[8] == "4.00" and r[10] == "1.000"  # VALU and MFMA instructions a weight
        assert r[11] == "10.0"                      # MFMA busy: 102400 / 1024000
        assert r[12] == "2.00" and r[13] == "25.0"  # waves a SIMD: 4 x 512000 / 1024000; waiting 128000 / 512000


def test_trace_summary_replays_and_floor(tmp_path):
    """bench.summarize_trace: the trace is cut into tokens at the head kernel (graph replays, eager tokens,
    floor replays, in that order, the first of each left out); per position the product's and the
    floor's mean durations and their difference come out as built, and the gap to the next kernel is
    the next begin minus this end."""
    run = tmp_path / "run"
    n, per = 4 * bench.LAYERS + 1, bench.TRACE_REPLAYS + 1
    head_grid = bench.VOCAB // 8 * 256
    pos = [("gemv_k<1, 8, 1, 4, 0>", 196608, 6.0), ("gemv_k<1, 8, 1, 4, 0>", 131072, 5.0), ("gemv_k<1, 4, 1, 4, 1>", 786432, 18.0),
           ("gemv_k<1, 8, 1, 12, 0>", 393216, 11.0)]
    rows, t = [], 10**6
    for mode in range(3):
        for _ in range(per):
            seq = [p for _ in range(bench.LAYERS) for p in pos] + [("gemv_k<1, 8, 1, 4, 0>", head_grid, 100.0)]
            for name, grid, us in seq:
                if mode == 2:
                    name, us = "read_k<8, 4, 0>", us - 0.5  # the floor: half a microsecond less everywhere
                rows.append({"Kernel_Name": f"void {name}(unsigned char const*, long)", "Grid_Size_X": grid, "Grid_Size_Y": 1,
                             "Grid_Size_Z": 1, "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
                t += int(us * 1000) + 250  # 0.25 us from each end to the next begin
            t += 10**6
    _csv(str(run / "ttrace" / "run_kernel_trace.csv"), ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp",
                                                         "End_Timestamp"], rows)
    line = {"token_trace": {"replays": bench.TRACE_REPLAYS, "products": n, "bytes_per_token": 7228294656,
                            **{k: {"ms_median": 1.4, "ms_min": 1.39} for k in ("graph", "eager", "floor")}}}
    (run / "ttrace.log").write_text("noise\n" + json.dumps(line) + "\n")
    out = tmp_path / "trace.md"
    bench.summarize_trace(str(run), out=str(out))
    text = out.read_text()
    table = [[c.strip() for c in l.split("|")[1:-1]] for l in text.split("## Product against its floor")[1].splitlines() if l.startswith("| ")]
    body = {r[0]: r for r in table[1:]}
    assert body["QKV 6144x4096"][1:4] == ["6.000", "5.500", "0.500"]
    assert body["gate+up 2x12288x4096"][1:5] == ["18.000", "17.500", "0.500", "16.0"]
    assert body["head 151936x4096"][1:5] == ["100.000", "99.500", "0.500", "0.5"]
    assert "0.250 us a boundary" in text
    assert f"products {bench.LAYERS * 40.0 + 100.0:.1f} us, floor {bench.LAYERS * 38.0 + 99.5:.1f} us" in text
