"""The inline-asm DMA of every kernel that uses dma.h (history, prefill, fused step and BF16
branch kernels) against the GFX9 hazard "a VALU write of an SGPR, then a vector-memory
instruction that reads it: 5 wait states", which the compiler checks for its own
instructions but not inside asm. The kernels are compiled to ISA here
(hipcc, no GPU) and every direct-to-LDS load is traced back, in straight-line order, to the
last writer of its SGPR operands (saddr base, M0): a VALU writer must be at least 5 wait
states (an `s_nop N` counts N + 1) before it.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _sgprs(tok):
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)}
    return {tok} if re.fullmatch(r"s\d+|m0", tok) else set()


def _late_sites(asm_text):
    """(kernel, writer, wait states, instruction) for every DMA read of a VALU-written SGPR
    fewer than 5 wait states after the write, in straight-line order within each kernel."""
    bad, history, kernel = [], [], None
    for line in asm_text.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            kernel, history = m.group(1), []
            continue
        ins = line.split(";")[0].strip()
        if not ins or ins.startswith(".") or ins.endswith(":") or kernel is None:
            continue
        parts = ins.replace(",", " ").split()
        op = parts[0]
        if op.startswith("global_load_lds"):
            reads = {"m0"} | (_sgprs(parts[2]) if len(parts) > 2 else set())
            waits = 0
            for w_op, w_dst, w_ws in reversed(history):
                if w_dst & reads:
                    if w_op.startswith("v_") and waits < 5:
                        bad.append((kernel, w_op, waits, ins))
                    break
                waits += w_ws
                if waits >= 5:
                    break
        nop = re.match(r"s_nop\s+(\d+)", ins)
        dst = _sgprs(parts[1]) if len(parts) > 1 else set()
        history.append((op, dst, int(nop.group(1)) + 1 if nop else 1))
    return bad


def test_scanner_flags_a_late_valu_base():
    # A planted case: the base written by v_readfirstlane two instructions before the DMA.
    text = """_Zk: ; @k
\tv_readfirstlane_b32 s6, v2
\tv_readfirstlane_b32 s7, v3
\ts_nop 0
\tglobal_load_lds_dwordx4 v4, s[6:7]
"""
    assert len(_late_sites(text)) == 1
    assert not _late_sites(text.replace("s_nop 0", "s_nop 4"))
    assert not _late_sites(text.replace("v_readfirstlane_b32 s7, v3", "s_mov_b32 s7, 0"))


# Every source whose kernels issue dma.h's direct-to-LDS loads, and a floor on how many
# loads each holds (so that a build that lost them does not pass vacuously).
DMA_SOURCES = {"history.hip": 100, "prefill.hip": 4, "step.hip": 4, "attention.hip": 4}


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc is not installed")
@pytest.mark.parametrize("source", sorted(DMA_SOURCES))
def test_kernels_keep_five_wait_states_before_every_dma(tmp_path, source):
    out = tmp_path / (Path(source).stem + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fno-gpu-flush-denormals-to-zero",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}",
           "--cuda-device-only", "-S", str(ROOT / "oscar_new_amd" / "csrc" / source), "-o",
           str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    text = out.read_text()
    assert text.count("global_load_lds_dword") >= DMA_SOURCES[source]
    assert _late_sites(text) == []
