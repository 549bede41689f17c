"""The chunked-prefill kernel's stream-K schedule, simulated on the CPU.

tests/pf_streamk_sim.cpp runs every workgroup's task loop with the kernel's own share
arithmetic (miniserve_amd/csrc/pf_streamk.h) over random task sizes and workgroup counts,
including work lists shorter than the workgroup count, and checks that every position is
taken once, that split tasks' partial slots are exactly those their merger reads, and that
the merger runs once all of them are in. A copy with the share count left unclamped (a
planted mistake: empty shares inside a task's contributor range) must fail it.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("pfsk") / "pf_streamk_sim"
    subprocess.run([gxx, "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'miniserve_amd' / 'csrc'}",
                    str(ROOT / "tests" / "pf_streamk_sim.cpp"), "-o", str(exe)], check=True)
    return exe


def run(exe, trials, mode):
    out = subprocess.run([str(exe), str(trials), str(mode)], check=True, capture_output=True,
                         text=True).stdout.split()
    return int(out[0]), int(out[1])


def test_schedule_covers_every_pair_once_and_merges_every_split_task(sim):
    violations, with_splits = run(sim, 20000, 0)
    assert with_splits > 10000
    assert violations == 0


def test_planted_unclamped_share_count_is_caught(sim):
    violations, _ = run(sim, 5000, 1)
    assert violations > 0
