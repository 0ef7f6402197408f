"""The prefill kernel's K-in-LDS path waits on hand-counted load counts
(prefill.hip: kBehindNext, v_next, kBehindLast). The compiler inserts no wait
of its own between a global_load_lds and the LDS read of its data, so the
counts are right only while every step issues its loads in the order they
assume: the two K tiles' direct-to-LDS loads (2 kDma per lane), then the two
V tiles' register loads (2 NJ), nothing in between. This compiles prefill.hip
for gfx950 (device code only, to assembly) and checks, for every K-in-LDS
kernel (D = 64 and 128), that

  - every run of K-tile DMA loads in program order is exactly 2 kDma
    global_load_lds_dwordx4 followed by 2 NJ global_load_dwordx2, and
  - the waits the source states are the ones emitted: vmcnt(2 NJ + 2 kDma
    + 2 NJ) before a step's K^T reads, vmcnt(2 kDma + 2 NJ) before its PV,
    vmcnt(2 NJ) for the last step,

with NJ = D / 16 and kDma = D * 16 * 2 / (64 * 16). A load reordered by a
compiler or code change makes one of these fail here, on the CPU, instead
of reading stale LDS on the GPU.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    from swiftllm_amd import build

    out = tmp_path_factory.mktemp("prefill_asm") / "prefill.s"
    cmd = [HIPCC, *build.FLAGS, "-x", "hip", "--cuda-device-only", "-S", "-o", str(out),
           str(build.CSRC / "prefill.hip")]
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    return out.read_text()


def _function(asm, D, fold):
    name = f"_ZN8swiftllm12_GLOBAL__N_120paged_prefill_kernelILi{D}ELb{int(fold)}ELb1EEEvNS0_11PrefillArgsE"
    m = re.search(r"^" + re.escape(name) + r":[^\n]*\n(.*?)\n\s*s_endpgm", asm, flags=re.S | re.M)
    assert m, f"no K-in-LDS prefill kernel for D={D} fold={fold}"
    return m.group(1)


def _vmem(body):
    ops = re.findall(r"^\s*((?:global|buffer)_(?:load|store|atomic)\w*)", body, flags=re.M)
    return ops


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("fold", [False, True])
def test_k_dma_loads_precede_v_loads_in_every_step(asm, D, fold):
    nj, kdma = D // 16, D * 16 * 2 // (64 * 16)
    ops = _vmem(_function(asm, D, fold))
    i, runs = 0, 0
    while i < len(ops):
        if ops[i] == "global_load_lds_dwordx4":
            run = ops[i:i + 2 * kdma + 2 * nj]
            assert run == ["global_load_lds_dwordx4"] * (2 * kdma) + ["global_load_dwordx2"] * (2 * nj), \
                f"D={D}: step loads out of order at VMEM op {i}: {run}"
            runs += 1
            i += len(run)
        else:
            i += 1
    assert runs >= 3, f"D={D}: expected the prologue, loop and tail steps, found {runs}"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("fold", [False, True])
def test_stated_wait_counts_are_emitted(asm, D, fold):
    nj, kdma = D // 16, D * 16 * 2 // (64 * 16)
    body = _function(asm, D, fold)
    waits = {int(v) for v in re.findall(r"s_waitcnt vmcnt\((\d+)\)", body)}
    for want, what in ((2 * nj + 2 * kdma + 2 * nj, "kBehindNext"), (2 * kdma + 2 * nj, "v_next"),
                       (2 * nj, "kBehindLast")):
        assert want in waits, f"D={D}: {what} = vmcnt({want}) not emitted (waits: {sorted(waits)})"
