"""The merge kernel's slot arithmetic on the CPU (miniserve_amd/csrc/merge_slots.h).

merge_slot_range turns the workspace header's layout words into the slots a merged row
reads. A header written for another geometry, or never written, must not send the merge
outside the workspace: tests/merge_slots_fuzz.cpp feeds it arbitrary header words, prefix
entries, rows and slot counts, and counts slots named at or past the workspace's end.
A copy without the final clamp (a planted mistake) must fail the same fuzz, so the fuzz
is shown to reach the out-of-range cases.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("slots") / "merge_slots_fuzz"
    subprocess.run([gxx, "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'miniserve_amd' / 'csrc'}",
                    str(ROOT / "tests" / "merge_slots_fuzz.cpp"), "-o", str(exe)], check=True)
    return exe


def run(exe, iters, mode):
    out = subprocess.run([str(exe), str(iters), str(mode)], check=True, capture_output=True,
                         text=True).stdout.split()
    return int(out[0]), int(out[1])


def test_every_named_slot_is_inside_the_workspace(fuzzer):
    violations, nonempty = run(fuzzer, 2_000_000, 0)
    assert nonempty > 100_000, "the fuzz must reach rows that do read partials"
    assert violations == 0


def test_planted_missing_clamp_is_caught(fuzzer):
    violations, _ = run(fuzzer, 200_000, 1)
    assert violations > 0
