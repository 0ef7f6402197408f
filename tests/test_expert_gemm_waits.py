"""The expert GEMM's hand-counted waits, checked in its gfx950 assembly.

moe_experts.hip loads its operand stages straight into LDS
(`buffer_load_dwordx4 ... lds`), which the compiler does not track, so two
waits are counted by hand:

  - moe_expert_gemm_kernel<GATED>: the weight group issues stage kt + 2 (8
    loads per lane) and then waits `vmcnt(8)` (kWaitLdsVm8), which must
    leave exactly those 8 in flight so that stage kt + 1 has landed before
    the barrier that hands it to the readers;
  - moe_expert_thin_kernel<GATED>: a ring of NS stages of L loads per lane
    with NS - 1 in flight; each step waits `vmcnt((NS - 2) * L)`, which must
    retire exactly the oldest stage. For 1, 2 and 4 tail tiles of 32 rows the
    stage holds the tile's 128 weight rows and 32 NTT tail rows (8 loads of
    16 bytes per row over 256 lanes), and the ring as many stages as fit in
    160 KiB.

This compiles moe_experts.hip for gfx950 (device code only, to assembly),
follows every path of each kernel (tests/asm_vmem.py) and checks what is in
flight at each of these waits. The checker itself is tested on the same
assembly with a load moved past a wait and with an extra load planted
before one: both must fail.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

import asm_vmem as av

HIPCC = "/opt/rocm/bin/hipcc"
THIN_LDS = 160 * 1024


def thin_shape(gated, ntt):
    """(loads per lane per stage L, ring stages NS) of a thin tile."""
    out = 64 if gated else 128
    tw = 2 * out if gated else out        # weight rows per stage
    rows = tw + 32 * ntt                  # plus the tail rows
    loads = rows * 8 // 256               # 16-byte chunks over 256 lanes
    stages = THIN_LDS // (rows * 64 * 2)  # stages of rows x 64 halves
    return loads, stages


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    from swiftllm_amd import build

    out = tmp_path_factory.mktemp("moe_asm") / "moe_experts.s"
    cmd = [HIPCC, *build.FLAGS, "-x", "hip", "--cuda-device-only", "-S", "-o", str(out),
           str(build.CSRC / "moe_experts.hip")]
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    return out.read_text()


def _body(asm, kernel, gated):
    return av.function_body(asm, av.mangled(kernel, f"Lb{int(gated)}E", "GemmArgs"))


def main_wait_errors(body, n=8):
    """Where a vmcnt(n) wait of the main kernel could leave anything other
    than the loads issued since the last barrier, all direct-to-LDS and n of
    them, in flight. Returns (waits found, error strings)."""
    w = av.walk(body)
    found, errs = 0, []
    for line, states in w.waits.items():
        for cnt, fly in states:
            if cnt != n:
                continue
            found += 1
            fresh = [e for e in fly if e[2]]
            if len(fresh) != n or any(k != "lds" for k, _, _ in fresh) or list(fly[-n:]) != fresh:
                errs.append(f"line {line}: {len(fresh)} ops since the barrier "
                            f"({[w.instr[l].split()[0] for _, l, _ in fresh]}), vmcnt({n})")
    return found, errs


def thin_wait_errors(body, gated):
    """Where a vmcnt(W > 0) wait of the thin kernel does not see exactly
    NS - 1 stages of direct-to-LDS loads in flight (so that it retires
    exactly the oldest stage) for one of the tile shapes. Returns (the
    (NTT, wait line) pairs matched, error strings)."""
    want = {}
    for ntt in (1, 2, 4):
        L, NS = thin_shape(gated, ntt)
        want.setdefault((NS - 2) * L, []).append((ntt, (NS - 1) * L))
    w = av.walk(body)
    matched, errs = set(), []
    for line, states in w.waits.items():
        for cnt, fly in states:
            if cnt == 0:
                continue
            if cnt not in want:
                errs.append(f"line {line}: vmcnt({cnt}) matches no thin tile shape")
                continue
            if any(k != "lds" for k, _, _ in fly):
                errs.append(f"line {line}: a vector memory op other than a stage load in flight")
            hit = [ntt for ntt, q in want[cnt] if q == len(fly)]
            if not hit:
                errs.append(f"line {line}: {len(fly)} loads in flight at vmcnt({cnt}), "
                            f"expected one of {[q for _, q in want[cnt]]}")
            matched.update((ntt, line) for ntt in hit)
    return matched, errs


@pytest.mark.parametrize("gated", [False, True])
def test_main_kernel_wait_leaves_only_the_new_stage(asm, gated):
    found, errs = main_wait_errors(_body(asm, "moe_expert_gemm_kernel", gated))
    assert found > 0, "no vmcnt(8) wait emitted (kWaitLdsVm8)"
    assert not errs, errs


@pytest.mark.parametrize("gated", [False, True])
def test_thin_kernel_waits_retire_exactly_one_stage(asm, gated):
    matched, errs = thin_wait_errors(_body(asm, "moe_expert_thin_kernel", gated), gated)
    assert not errs, errs
    assert {ntt for ntt, _ in matched} == {1, 2, 4}, f"tile shapes with a checked wait: {matched}"


def _move_load_past_wait(body, wait_re):
    """The body with the direct-to-LDS load just before the first wait
    matching wait_re moved to just after it."""
    body = list(body)
    wi = next(i for i, (_, t) in enumerate(body) if re.search(wait_re, t))
    li = max(i for i in range(wi) if "lds" in body[i][1] and av.VMEM.match(body[i][1]))
    load = body.pop(li)
    body.insert(wi, load)   # the wait moved up one place: the load now follows it
    return body


def _plant_load_before_wait(body, wait_re):
    body = list(body)
    wi = next(i for i, (_, t) in enumerate(body) if re.search(wait_re, t))
    body.insert(wi, (0, "global_load_dword v0, v[0:1], off"))
    return body


@pytest.mark.parametrize("plant", [_move_load_past_wait, _plant_load_before_wait])
def test_checker_fails_on_a_planted_mistake(asm, plant):
    body = plant(_body(asm, "moe_expert_gemm_kernel", True), r"vmcnt\(8\)")
    assert main_wait_errors(body)[1], "main kernel: planted mistake not caught"
    for gated in (False, True):
        L, NS = thin_shape(gated, 4)
        body = plant(_body(asm, "moe_expert_thin_kernel", gated), rf"vmcnt\({(NS - 2) * L}\)")
        assert thin_wait_errors(body, gated)[1], "thin kernel: planted mistake not caught"
