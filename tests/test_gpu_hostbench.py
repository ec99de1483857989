"""The C harness that times the host-pointer entry points (intel-phi-apl_amd/q8_hostbench, run by
bench.py for `configs.host_pointers`) runs to the end in a process of its own and prints one JSON
object: every section, with positive times and its calls' phases summing to no more than the
section's time. It times the entry points the reference's generated code calls
(src/card/rt.h:61-72); its results are timing only (the parity tests check the same calls' bits)."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOSTBENCH = os.path.join(ROOT, "intel-phi-apl_amd", "q8_hostbench")


@pytest.mark.parametrize("direct", ["1", "0"], ids=["x_direct", "x_copied"])
def test_hostbench_prints_every_section(direct):
    assert os.path.exists(HOSTBENCH), "q8_hostbench is not built (make -C intel-phi-apl_amd)"
    print("q8_hostbench 1", direct, flush=True)
    r = subprocess.run([HOSTBENCH, "1", direct], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    d = json.loads(r.stdout.strip().splitlines()[-1])
    assert d["x_direct"] == int(direct)
    for key, unit, per in (("rt_gemv_4096x4096", "us_per_call", "phases_per_call"), ("quartet_round_9b", "us_per_round", "phases_per_round"),
                           ("token_9b", "ms_per_token", "phases_per_token")):
        sec = d[key]
        assert sec[unit] > 0, key
        ph = sec[per]
        assert ph["calls"] > 0, key
        total_us = sec[unit] * (1000.0 if unit.startswith("ms") else 1.0)
        parts = ph["stage_x_us"] + ph["launch_us"] + ph["wait_us"] + ph["copy_out_us"]
        assert 0 < parts <= total_us * 1.05 + 1.0, (key, parts, total_us)
    assert d["token_9b"]["calls_per_token"] == 129
