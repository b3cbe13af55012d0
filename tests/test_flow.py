"""The single-launch kernels' task order and queue protocol, replayed on the
CPU (tests/c/flow_sim.cpp includes flash-cqt_amd/csrc/fcqt_flow.hpp, the
header the kernels use, built here with g++): every queue position decodes
to a distinct task, dependencies sit at earlier positions, and simulated
persistent workgroups with random task durations always finish, at 1 to 600
workgroups per queue and every batch shape tried; a planted order with the
lags reversed must fail."""
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_flow_order_and_protocol(tmp_path):
    exe = tmp_path / "flow_sim"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-Werror",
                    str(ROOT / "tests" / "c" / "flow_sim.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.split("\n")
    assert lines[0].startswith("planted: FAIL"), r.stdout     # the planted order was caught
    assert lines[1].startswith("ok ") and int(lines[1].split()[1]) >= 5000, r.stdout
