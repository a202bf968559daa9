"""Invariants of the generated gfx950 code that the kernels' inline assembly
relies on (CPU-only: hipcc cross-compiles to assembly without a GPU)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "lighthouse-attention_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


def _device_asm(src, tmp_path):
    out = tmp_path / "dev.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", "-I" + CSRC, "--cuda-device-only", "-S", "-o", str(out),
                    os.path.join(CSRC, src)], check=True, capture_output=True)
    return out.read_text()


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None, reason="hipcc not available")
def test_m0_only_in_inline_asm(tmp_path):
    """The direct global->LDS loads set M0 inside inline assembly.  M0 is a
    reserved register the compiler may assume unchanged across an asm
    statement, so no compiler-generated instruction may use it."""
    asm = _device_asm("lh_attn.hip", tmp_path)
    inside, in_asm, outside = 0, False, []
    for line in asm.split("\n"):
        if ";;#ASMSTART" in line:
            in_asm = True
        elif ";;#ASMEND" in line:
            in_asm = False
        elif re.search(r"\bm0\b", line.split(";")[0]):
            if in_asm:
                inside += 1
            else:
                outside.append(line.strip())
    assert inside > 0, "expected the inline-asm direct loads to set M0"
    assert not outside, f"compiler-generated M0 uses: {outside[:5]}"


SOURCES = ["lh_attn.hip", "lh_select.hip", "lh_pyramid.hip", "lh_scatter.hip", "lh_model.hip"]


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None, reason="hipcc not available")
@pytest.mark.parametrize("src", SOURCES)
def test_no_register_spills(src, tmp_path):
    """No kernel of the library spills registers to scratch (a spill inside the
    attention kernels' step loops costs a memory round trip per step)."""
    asm = _device_asm(src, tmp_path)
    kernels, name = {}, None
    for line in asm.split("\n"):
        m = re.match(r"\s+\.(name|private_segment_fixed_size|vgpr_spill_count):\s+(\S+)", line)
        if not m:
            continue
        if m.group(1) == "name":
            name = m.group(2)
            kernels[name] = [None, None]
        elif name is not None:
            kernels[name][0 if m.group(1) == "private_segment_fixed_size" else 1] = int(m.group(2))
    kernels = {k: tuple(v) for k, v in kernels.items() if v[0] is not None and v[1] is not None}
    assert kernels, "no kernel metadata found"
    bad = {k: v for k, v in kernels.items() if v != (0, 0)}
    assert not bad, f"kernels with scratch (private bytes, spilled VGPRs): {bad}"
