"""The CPU test suite under AddressSanitizer and UndefinedBehaviorSanitizer.

    python -m swiftllm_amd.sanitize          # build, then run pytest -m "not gpu"

Builds, in their own directories:
  - libswiftllm_hip.so and libswiftllm_ceilings.so with the host code (the C
    ABI: argument validation, slot mapping, block-table packing, the
    size_t -> int32 narrowing of the params twins, launch set-up) compiled
    with -fsanitize=address,undefined; the device code is built as usual
    (each -fsanitize= sits behind -Xarch_host, so it applies to the host
    pass only);
  - oracle/_sanitize/liboracle.so (`make -C oracle sanitize`), the C oracle
    with the same sanitizers;
then runs the CPU tests with those libraries (SWIFTLLM_HIP_LIB,
SWIFTLLM_CEILINGS_LIB, SWIFTLLM_ORACLE_LIB) and the shared clang ASan runtime
preloaded into the interpreter. Leak checking is off (the interpreter itself
is not instrumented); any other report fails the run.

CPU only: nothing here runs on a GPU, and a GPU box never builds or loads
these libraries.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

from . import build as hip_build

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
OUT = PKG / "_sanitize"
OBJ = hip_build.CSRC / "_build_sanitize"
CLANG = "/opt/rocm/llvm/bin/clang"

HOST_SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-sanitize-recover=undefined",
                 "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]


def asan_runtime() -> str:
    out = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], check=True,
                         stdout=subprocess.PIPE, text=True).stdout.strip()
    if not Path(out).exists():
        raise FileNotFoundError(f"clang ASan runtime not found ({out})")
    return out


def build() -> dict:
    """Builds the sanitized libraries; returns the environment that selects them."""
    OUT.mkdir(exist_ok=True)
    OBJ.mkdir(parents=True, exist_ok=True)
    libs = {"libswiftllm_hip.so": hip_build.SOURCES, "libswiftllm_ceilings.so": hip_build.CEILINGS_SOURCES}
    for src in hip_build.SOURCES + hip_build.CEILINGS_SOURCES:
        hip_build._run([hip_build.HIPCC, *hip_build.FLAGS, *HOST_SANITIZE, "-x", "hip", "-c",
                        str(hip_build.CSRC / src), "-o", str(OBJ / (src + ".o"))])
    for name, sources in libs.items():
        hip_build._run([hip_build.HIPCC, "-shared", "-fPIC", f"--offload-arch={hip_build.ARCH}",
                        "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                        "-shared-libasan", *[str(OBJ / (s + ".o")) for s in sources],
                        "-Wl,-rpath,/opt/rocm/lib", "-o", str(OUT / name)])
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize"], check=True)
    return {
        "SWIFTLLM_HIP_LIB": str(OUT / "libswiftllm_hip.so"),
        "SWIFTLLM_CEILINGS_LIB": str(OUT / "libswiftllm_ceilings.so"),
        "SWIFTLLM_ORACLE_LIB": str(ROOT / "oracle" / "_sanitize" / "liboracle.so"),
        "LD_PRELOAD": asan_runtime(),
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
    }


def run(pytest_args: list[str]) -> int:
    env = dict(os.environ, **build())
    cmd = [sys.executable, "-m", "pytest", str(ROOT / "tests"), "-q", "-m", "not gpu", *pytest_args]
    print(" ".join(f"{k}={v}" for k, v in env.items() if k.startswith(("SWIFTLLM_", "LD_PRE", "ASAN", "UBSAN"))),
          file=sys.stderr)
    return subprocess.run(cmd, env=env, cwd=str(ROOT)).returncode


if __name__ == "__main__":
    sys.exit(run(sys.argv[1:]))
