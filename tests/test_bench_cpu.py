"""bench.py pieces that run without a GPU: the single-GPU refusal, strict
JSON, and the host-core baseline's contract on a tiny sample."""
import json
import math
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2
    assert "single-GPU" in r.stderr and r.stdout == ""


@pytest.fixture(scope="module")
def bench():
    sys.path.insert(0, str(ROOT))
    import bench as b
    return b


def test_json_safe_is_strict(bench):
    v = bench.json_safe({"a": float("inf"), "b": [1.0, float("nan")], "c": {"d": 2}})
    assert v == {"a": "inf", "b": [1.0, "nan"], "c": {"d": 2}}
    json.loads(json.dumps(v, allow_nan=False))


def test_cpu_baseline_contract(bench):
    """kind "port", os.cpu_count() threads (uncapped, restored afterwards),
    the CPU model and affinity, a sample description, the batch-64 value
    plus batches 1, 4 and 16 (run here at batch 2 on a tiny budget)."""
    import os
    import torch
    before = torch.get_num_threads()
    cb = bench.cpu_baseline(batch=2, budget_s=0.01, budget_b1_s=0.01, max_reps=1)
    assert torch.get_num_threads() == before
    assert cb["kind"] == "port" and cb["unit"] == "slice round trips/s"
    assert cb["cores"] == os.cpu_count() and cb["value"] > 0 and "round trips" in cb["sample"]
    assert "cpus_in_affinity" in cb and "cpu_model" in cb
    assert set(cb["per_batch"]) == {"1", "2", "4", "16"}
    assert cb["snr_db"] > 125 and cb["batch1"]["snr_db"] > 125
    assert all(math.isfinite(v["round_trips_per_s"]) for v in cb["per_batch"].values())
