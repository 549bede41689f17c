"""Build libmsattn.so (gfx950) in-tree with hipcc.

Usage: ``python -m miniserve_amd.build [--define NAME=VALUE ...]`` (or
``__graft_entry__.build()``). Every ``csrc/*.hip`` file is compiled to an object
under ``_build/`` in parallel, then linked into ``miniserve_amd/libmsattn.so``,
which the Python package loads with ctypes. A build always recompiles: nothing
is cached across calls. ``--define`` overrides one of the compile-time tuning
knobs (the ``MSATTN_*`` macros of csrc/) for a measurement build; rebuild
without it to restore the defaults.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD_DIR = PKG / "_build"
LIB_PATH = PKG / "libmsattn.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops keeps the compiler from emitting v_pk_{add,mul,fma}_f32.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{CSRC}",
    f"-I{INCLUDE}",
]


# Per-file extra flags. The prefill kernel keeps its MFMA accumulators in ordinary VGPRs:
# it needs 244 registers that way, while the default accumulator-register form spends
# about 220 copy instructions per 64-key step moving scores and outputs between the two
# register files.
FILE_FLAGS = {
    "prefill_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "prefill_mfma_fp8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "prefill_mfma_f32kv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = True, jobs: int | None = None,
          defines: list[str] | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libmsattn.so; returns its path.
    `defines`: NAME=VALUE overrides of MSATTN_* tuning macros."""
    extra = []
    for d in defines or []:
        name = d.split("=", 1)[0]
        if not name.startswith("MSATTN_") or not name.replace("_", "").isalnum():
            raise ValueError(f"--define takes MSATTN_* tuning macros, not {d!r}")
        extra.append(f"-D{d}")
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; the msattn library needs ROCm's hipcc")
    hipcc = HIPCC if Path(HIPCC).exists() else shutil.which("hipcc")
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))

    def compile_one(pair):
        src, obj = pair
        if verbose:
            print(f"[msattn build] hipcc {src.name}", flush=True)
        _run([hipcc, *COMMON_FLAGS, *extra, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o",
              str(obj)])

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, zip(sources, objs)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[msattn build] wrote {LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="build libmsattn.so for gfx950")
    ap.add_argument("--define", action="append", default=[], metavar="MSATTN_NAME=VALUE",
                    help="override a compile-time tuning macro (measurement builds)")
    build(defines=ap.parse_args().define)
