"""Build libswiftllm_hip.so in-tree with hipcc for gfx950.

    python -m swiftllm_amd.build          # or swiftllm_amd.build.build()

Every HIP source under csrc/ is compiled to an object in csrc/_build/ and
linked into swiftllm_amd/libswiftllm_hip.so (the path) or
swiftllm_amd/libswiftllm_ceilings.so (measurement kernels) next to this file,
so the libraries travel with the source tree.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = CSRC / "_build"
LIB = PKG / "libswiftllm_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["abi.cpp", "paged_attention.hip", "prefill.hip", "cache_ops.hip", "block_copy.hip", "moe.hip",
           "moe_experts.hip", "checks.hip"]

# The measurement kernels bench.py times beside the path (include/swiftllm_ceilings.h)
# are a library of their own, outside the drop-in interface.
CEILINGS_LIB = PKG / "libswiftllm_ceilings.so"
CEILINGS_SOURCES = ["ceilings.hip"]

FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # No packed-fp32 instructions in generated device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-I", str(ROOT / "include"),
    "-I", str(CSRC),
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _link(lib: Path, sources: list[str], verbose: bool) -> None:
    tmp = lib.with_suffix(".so.tmp")
    link = [
        HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}",
        *[str(OBJ / (s + ".o")) for s in sources],
        "-Wl,-rpath,/opt/rocm/lib", "-o", str(tmp),
    ]
    if verbose:
        print(" ".join(link))
    _run(link)
    os.replace(tmp, lib)


def build(verbose: bool = False) -> Path:
    """Compile every source and link both shared libraries; returns the path
    of libswiftllm_hip.so."""
    OBJ.mkdir(parents=True, exist_ok=True)
    jobs = []
    for src in SOURCES + CEILINGS_SOURCES:
        obj = OBJ / (src + ".o")
        lang = ["-x", "hip"]
        jobs.append([HIPCC, *FLAGS, *lang, "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 4)) as ex:
        for cmd in jobs:
            if verbose:
                print(" ".join(cmd))
        list(ex.map(_run, jobs))
    _link(LIB, SOURCES, verbose)
    _link(CEILINGS_LIB, CEILINGS_SOURCES, verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
