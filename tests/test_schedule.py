"""Tile scheduler of the persistent kernel, checked on the host (no GPU).

tests/sched_check.cpp compiles the kernel's own scheduler header (gg_schedule.h) with g++
and checks bijection, per-XCD contiguity, band locality and full coverage of the kernel's
tile walk, including ragged and empty groups.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "groupgemm-cktile-optimized_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_scheduler_properties(tmp_path):
    exe = tmp_path / "sched_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-Wall", "-I", CSRC, os.path.join(HERE, "sched_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "schedule OK" in r.stdout
