"""The product kernels' MFMA code is free of the hazards the compiler cannot see.

The products issue MFMAs from inline asm; the compiler's hazard recognizer does not look into
it, so a register copy the compiler places next to an MFMA gets no wait states. One such
copy (accumulators moved between AGPRs right after the MFMA that wrote them, in the B X
kernel's beta steps) made B X differ by an ulp from run to run; another (accumulators
permuted between registers where the loop before the peeled beta K-tiles exits, 10 wait states
after the last MFMA) only showed once the scan followed branches. This test compiles gemm.hip
for gfx950 to assembly and scans every kernel that issues MFMAs (mfma_hazards.py): no VALU
access to an MFMA's result within its latency, no MFMA reading a register a VALU op wrote
within 3 wait states."""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIPCC = "/opt/rocm/bin/hipcc"
sys.path.insert(0, HERE)
import mfma_hazards  # noqa: E402


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")
def test_product_kernels_have_no_mfma_hazards(tmp_path):
    asm = tmp_path / "gemm.s"
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-fPIC", "-Wno-unused-function",
           "-Wno-int-to-pointer-cast", "-Wno-inline-asm", "-mllvm",
           "-pragma-unroll-threshold=1000000", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I" + os.path.join(ROOT, "include"), "--cuda-device-only", "-S",
           os.path.join(ROOT, "dtensor-muon_amd", "csrc", "gemm.hip"), "-o", str(asm)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=900)
    found = {}
    for name, lines in mfma_hazards.kernels(str(asm)):
        if any("v_mfma" in line for line in lines):
            found[name] = mfma_hazards.scan(lines)
    assert any("nn16" in n for n in found) and any("s16" in n for n in found)
    bad = {n: v[:3] for n, v in found.items() if v}
    assert not bad, bad


_M = "v_mfma_f32_32x32x16_bf16 v[0:15], v[16:19], v[20:23], v[0:15]"
_NOPS = ["s_nop 7", "s_nop 7", "s_nop 7"]


@pytest.mark.parametrize("name, code, hazards", [
    ("straight line", [_M, "v_mov_b32_e32 v40, v3"], 1),
    ("enough wait states", [_M] + _NOPS + ["v_mov_b32_e32 v40, v3"], 0),
    ("falls through a label", [_M, ".LBB0_1:", "v_mov_b32_e32 v40, v3"], 1),
    ("label reached by a jump only",
     [_M, "s_branch .LBB0_2", ".LBB0_1:", "v_mov_b32_e32 v40, v3", ".LBB0_2:", "s_endpgm"], 0),
    ("taken forward branch",
     [_M, "s_cbranch_scc1 .LBB0_2"] + _NOPS + [".LBB0_2:", "v_mov_b32_e32 v40, v3"], 1),
    ("loop back-edge",
     [".LBB0_1:", "v_mov_b32_e32 v40, v3"] + _NOPS + [_M, "s_cbranch_scc1 .LBB0_1", "s_endpgm"], 1),
    ("VALU write read by an MFMA", ["v_mov_b32_e32 v16, 0", _M], 1),
    ("MFMA chain on one accumulator", [_M, _M], 0),
])
def test_scanner_follows_control_flow(name, code, hazards):
    """The scanner itself, on hand-written snippets: hazards across fallthrough, taken
    branches and loop back-edges are found; a block reached only by a jump from elsewhere
    does not inherit the state before it."""
    assert len(mfma_hazards.scan([line + "\n" for line in code])) == hazards, name
