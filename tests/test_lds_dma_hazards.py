"""Wait-state check of the HBM -> LDS copies in the compiled kernels (CPU only, needs hipcc).

The attention kernels issue `global_load_lds_dwordx4` as inline assembly, which the compiler's
hazard recognizer does not inspect. On gfx9-family GPUs (gfx950 included) a VALU instruction that
writes an SGPR (v_readlane of a spilled SGPR, v_readfirstlane, v_cmp) needs 5 wait states before a
vector memory instruction reads that SGPR; the copies read their SGPR base pair and M0. Without
them the copy can use a stale base address. This test compiles the kernel sources exactly as the
Makefile does, to gfx950 assembly, and checks every LDS DMA: within the 5 wait states before it, in
its basic block, the last writer of each SGPR it reads (base pair, M0) is not a VALU instruction.
The inline copies make that so by construction: the compiler writes M0 with an SALU move, and the
SGPR base is moved by the SALU inside the asm.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "amd-incstinct-labs_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["prefill.hip", "decode.hip", "gemm.hip"]


def _flags(src):
    f = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-I../include", "-Icsrc", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument"]
    if src in ("prefill.hip", "decode.hip"):
        f += ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]
    return f


def _sgprs(text):
    regs = set()
    for m in re.finditer(r"\bs\[(\d+):(\d+)\]", text):
        regs |= {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    regs |= set(re.findall(r"(?<![\w\[:])s\d+\b", text))
    if re.search(r"\bm0\b", text):
        regs.add("m0")
    return regs


def dma_hazards(asm_lines):
    """(index, text) of every LDS DMA that may read an SGPR (its base pair or M0) written by a VALU
    instruction fewer than 5 wait states earlier. Walking back through the DMA's basic block, an
    SALU write of a register ends the check for that register; reaching the top of the block with
    registers still unchecked and fewer than 5 wait states counts as a hazard."""
    insts = []
    for raw in asm_lines:
        s = raw.split(";")[0].strip()
        if not s:
            continue
        if re.match(r"^[.\w$]+:$", s):
            insts.append(("label", s))
        elif not s.startswith("."):
            insts.append(("inst", s))
    bad = []
    for i, (kind, s) in enumerate(insts):
        if kind != "inst" or not s.startswith("global_load_lds"):
            continue
        operands = s.split(None, 1)[1].split(",")
        reads = {"m0"} | (_sgprs(operands[1]) if len(operands) > 1 else set())
        ws, ok = 0, False
        for j in range(i - 1, -1, -1):
            k, t = insts[j]
            if k == "label":
                break
            parts = t.split(None, 1)
            op = parts[0]
            dst = _sgprs(parts[1].split(",")[0]) if len(parts) > 1 else set()
            if op == "s_nop":
                ws += int(parts[1], 0) + 1
            elif op.startswith("v_") and dst & reads:
                break
            else:
                if op.startswith("s_") and dst & reads:
                    reads -= dst          # the latest writer is the SALU: no wait states needed
                ws += 1
            if ws >= 5 or not reads:
                ok = True
                break
        if not ok:
            bad.append((i, s))
    return bad


def test_dma_hazard_scan_catches_a_valu_sgpr_write():
    # the pattern of the fault this test guards against, and the guarded form
    assert dma_hazards(["v_readlane_b32 s16, v255, 31", "v_readlane_b32 s17, v255, 32", "s_nop 0",
                        "global_load_lds_dwordx4 v241, s[16:17]"])
    assert dma_hazards(["v_readfirstlane_b32 m0, v3", "s_nop 0", "global_load_lds_dwordx4 v[2:3], off"])
    assert dma_hazards([".LBB0_1:", "s_nop 0", "global_load_lds_dwordx4 v[2:3], off"])
    assert not dma_hazards(["v_readlane_b32 s16, v255, 31", "v_readlane_b32 s17, v255, 32", "s_nop 4",
                            "global_load_lds_dwordx4 v241, s[16:17]"])
    assert not dma_hazards([".LBB0_1:", "s_mov_b32 m0, s4", "s_nop 4", "global_load_lds_dwordx4 v[2:3], off"])
    # the form dma16_s emits: the base moved by the SALU into a pair only the copy reads
    assert not dma_hazards(["v_readlane_b32 s16, v255, 31", "v_readlane_b32 s17, v255, 32", "s_mov_b32 m0, s2",
                            "s_mov_b64 s[20:21], s[16:17]", "s_nop 0", "global_load_lds_dwordx4 v241, s[20:21]"])
    assert not dma_hazards([".LBB0_1:", "s_mov_b32 m0, s4", "s_nop 0", "global_load_lds_dwordx4 v[2:3], off"])
    assert dma_hazards([".LBB0_1:", "s_mov_b32 m0, s4", "s_nop 0", "global_load_lds_dwordx4 v2, s[20:21]"])


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src", SOURCES)
def test_lds_dma_wait_states(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = [HIPCC] + _flags(src) + ["--offload-device-only", "-S", os.path.join("csrc", src), "-o", str(out)]
    r = subprocess.run(cmd, cwd=PKG, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = out.read_text().split("\n")
    n_dma = sum(1 for l in lines if l.strip().startswith("global_load_lds"))
    assert n_dma > 0
    bad = dma_hazards(lines)
    assert not bad, f"{len(bad)} LDS DMA(s) without 5 wait states after a VALU SGPR write, e.g. {bad[:3]}"
