"""Static checks of the hand-written instructions in the matmul and attention kernels (no GPU needed).

The VALU fallback matmul's FMAs with the DPP64 modifier row_newbcast sit in inline assembly, so the compiler's hazard recognizer
does not see them. The CDNA rule they must obey: a DPP instruction comes at least two wait states after any vector
ALU write of a VGPR it reads (the previous instruction and `s_nop n` count 1 and n + 1 states). This test compiles
the two kernel sources to gfx950 assembly with the library's own flags and walks back from every DPP instruction.

The matrix-core matmul's and attention kernels' stage copies are inline-assembly memory loads whose base address is an SGPR pair. A vector
ALU instruction that writes an SGPR (readfirstlane, readlane, a compare into an SGPR pair) must come at least five
wait states before a memory instruction that reads it; the same walk-back checks that rule for every load that names
an SGPR base.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from etalii_dllm_amd import build as B

SOURCES = ["gemm.hip", "attn_lds.hip"]


def _regs(token: str) -> set[int]:
    m = re.match(r"v\[(\d+):(\d+)\]", token)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", token)
    return {int(m.group(1))} if m else set()


def _instructions(asm: str) -> list[str]:
    out = []
    for line in asm.splitlines():
        line = line.split(";")[0].strip()
        if not line or line.startswith(".") or line.endswith(":"):
            continue
        out.append(line)
    return out


def dpp_hazards(asm: str) -> tuple[int, list[str]]:
    lines = _instructions(asm)
    checked, bad = 0, []
    for idx, line in enumerate(lines):
        if "_dpp" not in line.split()[0]:
            continue
        checked += 1
        operands = [o.strip().split()[0] for o in line.split(None, 1)[1].split(",")]
        read = set().union(*(_regs(o) for o in operands))  # the destination too: v_fmac reads it
        states, j = 0, idx - 1
        while j >= 0 and states < 2:
            parts = lines[j].split(None, 1)
            if parts[0] == "s_nop":
                states += int(parts[1]) + 1
            else:
                if parts[0].startswith("v_") and len(parts) > 1 and _regs(parts[1].split(",")[0].strip()) & read:
                    bad.append(f"{lines[j]}  ->  {line}")
                states += 1
            j -= 1
    return checked, bad


def _sregs(token: str) -> set[int]:
    m = re.match(r"s\[(\d+):(\d+)\]", token)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", token)
    return {int(m.group(1))} if m else set()


def sgpr_base_hazards(asm: str) -> tuple[int, list[str]]:
    """Memory instructions reading an SGPR base fewer than 5 wait states after a vector ALU write of it."""
    lines = _instructions(asm)
    checked, bad = 0, []
    for idx, line in enumerate(lines):
        op = line.split()[0]
        if not (op.startswith("global_") or op.startswith("buffer_")) or len(line.split(None, 1)) < 2:
            continue
        read = set().union(*(_sregs(o.strip().split()[0]) for o in line.split(None, 1)[1].split(",")))
        if not read:
            continue
        checked += 1
        states, j = 0, idx - 1
        while j >= 0 and states < 5:
            parts = lines[j].split(None, 1)
            if parts[0] == "s_nop":
                states += int(parts[1]) + 1
            else:
                if parts[0].startswith("v_") and len(parts) > 1 and _sregs(parts[1].split(",")[0].strip()) & read:
                    bad.append(f"{lines[j]}  ->  {line}")
                states += 1
            j -= 1
    return checked, bad


def _device_asm(tmp_path, source):
    asm = tmp_path / (source + ".s")
    cmd = [B.HIPCC, *B.FLAGS, "--cuda-device-only", "-S", str(B.CSRC / source), "-o", str(asm)]
    result = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stderr[-2000:]
    return asm.read_text()


@pytest.mark.skipif(not Path(B.HIPCC).exists() and shutil.which("hipcc") is None, reason="hipcc not available")
@pytest.mark.parametrize("source", SOURCES)
def test_hand_written_instructions_respect_their_wait_states(tmp_path, source):
    asm = _device_asm(tmp_path, source)
    dpp_checked, bad = dpp_hazards(asm)
    assert not bad, f"{len(bad)} DPP hazards, e.g. {bad[:3]}"
    sgpr_checked, bad = sgpr_base_hazards(asm)
    assert not bad, f"{len(bad)} SGPR-base hazards, e.g. {bad[:3]}"
    assert dpp_checked + sgpr_checked > 0  # the walk found the hand-written instructions it is meant to check


def test_the_checkers_find_a_hazard():
    asm = "v_cvt_f64_f32_e32 v[4:5], v1\nv_fmac_f64_dpp v[8:9], v[2:3], v[4:5] row_newbcast:1\n"
    assert dpp_hazards(asm)[1]
    assert not dpp_hazards("v_cvt_f64_f32_e32 v[4:5], v1\ns_nop 1\nv_fmac_f64_dpp v[8:9], v[2:3], v[4:5] row_newbcast:1\n")[1]
    load = "v_readfirstlane_b32 s87, v1\nv_readfirstlane_b32 s86, v0\ns_nop 0\nglobal_load_lds_dwordx4 v191, s[86:87]\n"
    assert sgpr_base_hazards(load)[1]
    assert not sgpr_base_hazards(load.replace("s_nop 0", "s_nop 4"))[1]
