"""bench.py's host-side contract, on the CPU: the one-GPU refusal, the steps captured
per graph, and the cpu_baseline object (the oracle's SDPA restatement on a bounded
sample of the same workload)."""
import argparse
import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from miniserve_amd.workloads import make_workload  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


@pytest.mark.parametrize("steps,graph_steps,want", [
    (200, 0, 10), (13, 0, 1), (12, 0, 6), (7, 0, 7), (20, 4, 4)])
def test_steps_per_graph(steps, graph_steps, want):
    assert bench.graph_steps(argparse.Namespace(steps=steps, graph_steps=graph_steps)) == want


def test_graph_steps_must_divide_the_steps():
    with pytest.raises(SystemExit):
        bench.graph_steps(argparse.Namespace(steps=10, graph_steps=3))


def test_cpu_baseline_object():
    cpu = torch.device("cpu")
    w = make_workload(1, device=cpu, values_device=cpu, layers=1, part="decode")
    r = bench.cpu_baseline(w, 0.05)
    assert set(r) >= {"value", "unit", "cores", "kind", "sample"}
    assert r["kind"] == "port" and r["unit"] == "GB/s" and r["value"] > 0
    assert r["cores"] >= 1 and "C1" in r["sample"]
    assert r["cpu_model"] and r["cpu_model"] != "unknown"


def test_library_hash_names_the_loaded_library():
    h = bench.library_sha256()
    assert len(h) == 16 and int(h, 16) >= 0
