"""The tiled 16x16x32 kernel keeps its 256 fp32 accumulators in fixed AGPRs
reached only through inline assembly (reframework_amd/csrc/acc_regs.h). That
is sound only while the compiler itself leaves the AGPRs alone (no spills into
them, no MFMAs of its own) and keeps the operand fragments in registers. This
compiles ffn_tiled.hip to gfx950 assembly (no GPU needed) and checks both in
every instance of ffn_tiled16_kernel; it also checks that acc_regs.h is what
its generator writes."""

from __future__ import annotations

import os
import re
import subprocess
import sys

import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "reframework_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def test_acc_regs_header_matches_generator():
    out = subprocess.run([sys.executable, os.path.join(CSRC, "gen_acc_regs.py")], capture_output=True,
                         text=True, check=True).stdout
    with open(os.path.join(CSRC, "acc_regs.h")) as f:
        assert f.read() == out


def _tiled_flags():
    """The extra flags the Makefile gives ffn_tiled.hip."""
    with open(os.path.join(CSRC, "Makefile")) as f:
        m = re.search(r"^TILED_FLAGS := (.*)$", f.read(), re.M)
    assert m, "Makefile lost TILED_FLAGS"
    return m.group(1).split()


def test_makefile_forbids_vgpr_spills_to_agprs():
    flags = _tiled_flags()
    assert "-amdgpu-spill-vgpr-to-agpr=0" in flags
    with open(os.path.join(CSRC, "Makefile")) as f:
        assert "$(OBJDIR)/ffn_tiled.o: HIPFLAGS += $(TILED_FLAGS)" in f.read()


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_tiled16_accumulators_stay_in_their_agprs(tmp_path):
    asm = tmp_path / "ffn_tiled.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", *_tiled_flags(), "--cuda-device-only", "-S",
                    os.path.join(CSRC, "ffn_tiled.hip"), "-o", str(asm)],
                   check=True, capture_output=True, cwd=CSRC)
    lines = asm.read_text().splitlines()
    starts = [i for i, l in enumerate(lines) if re.match(r"^_Z\S*ffn_tiled16_kernel\S*:", l)]
    assert len(starts) == 8  # bf16 / f16 x gate_up / down x ragged or not
    for st in starts:
        name = lines[st].split(":")[0]
        end = next(i for i in range(st, len(lines)) if "s_endpgm" in lines[i])
        in_asm = False
        for l in lines[st:end]:
            if "ASMSTART" in l:
                in_asm = True
            elif "ASMEND" in l:
                in_asm = False
            elif not in_asm:
                code = l.split(";")[0]
                assert not re.search(r"\ba\[?\d", code), f"{name}: compiler-generated AGPR use: {l.strip()}"
                assert "scratch_" not in code, f"{name}: scratch access: {l.strip()}"
        meta = "\n".join(l for l in lines if l.strip().startswith(f".set {name}."))
        assert re.search(rf"{re.escape(name)}\.num_agpr, 256\b", meta), name
        assert re.search(rf"{re.escape(name)}\.private_seg_size, 0\b", meta), name
