"""Every host wait of the library ends: the wait loop (intel-phi-apl_amd/csrc/q8_wait.h), driven on
the CPU by tests/c/wait_deadline.cpp with polls that complete at once, after 50 ms, or never. A wait
that never completes prints what it waited for and ends the process with status 3 at its deadline,
as the reference's card does without its host (src/card/link.c:17-32); the others return."""
import os
import subprocess
import time

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("wait") / "wait_deadline")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "intel-phi-apl_amd", "csrc"),
                    os.path.join(ROOT, "tests", "c", "wait_deadline.cpp"), "-o", exe], check=True)
    return exe


def test_wait_returns_when_done(driver):
    r = subprocess.run([driver, "done", "5"], capture_output=True, text=True, timeout=30)
    assert r.returncode == 0, r.stderr
    assert "returned after 1000 polls" in r.stdout


def test_wait_returns_after_sleeping_polls(driver):
    r = subprocess.run([driver, "slow", "5"], capture_output=True, text=True, timeout=30)
    assert r.returncode == 0, r.stderr
    assert "returned after" in r.stdout


@pytest.mark.parametrize("deadline", [0.2, 1.0])
def test_wait_never_done_exits_3_at_deadline(driver, deadline):
    t0 = time.monotonic()
    r = subprocess.run([driver, "never", str(deadline)], capture_output=True, text=True, timeout=30)
    took = time.monotonic() - t0
    assert r.returncode == 3, (r.returncode, r.stdout, r.stderr)
    assert "returned" not in r.stdout
    assert "the never case did not complete within" in r.stderr and "exiting with status 3" in r.stderr
    assert deadline <= took < deadline + 2.0, took
