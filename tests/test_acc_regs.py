"""The tiled 16x16x32 kernel keeps its 256 fp32 accumulators in fixed AGPRs
reached only through inline assembly (reframework_amd/csrc/acc_regs.h). That
is sound only while the compiler itself leaves the AGPRs alone (no spills into
them, no MFMAs of its own) and keeps the operand fragments in registers. This
compiles ffn_tiled16.hip to gfx950 assembly (no GPU needed) as each of the
Makefile's instances and checks both in every ffn_tiled16_kernel; it also
checks that acc_regs.h is what its generator writes."""

from __future__ import annotations

import concurrent.futures
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
    """The extra flags the Makefile gives the tiled kernels."""
    with open(os.path.join(CSRC, "Makefile")) as f:
        m = re.search(r"^TILED_FLAGS := (.*)$", f.read(), re.M)
    assert m, "Makefile lost TILED_FLAGS"
    return m.group(1).split()


def _tiled16_instances():
    """The (dtype, projection) instances the Makefile builds ffn_tiled16.hip as."""
    with open(os.path.join(CSRC, "Makefile")) as f:
        m = re.search(r"^TILED16 := (.*)$", f.read(), re.M)
    assert m, "Makefile lost TILED16"
    return m.group(1).split()


def test_makefile_forbids_vgpr_spills_to_agprs():
    flags = _tiled_flags()
    assert "-amdgpu-spill-vgpr-to-agpr=0" in flags
    with open(os.path.join(CSRC, "Makefile")) as f:
        mk = f.read()
    assert "$(OBJDIR)/ffn_tiled.o: HIPFLAGS += $(TILED_FLAGS)" in mk
    assert "$(HIPCC) $(HIPFLAGS) $(TILED_FLAGS) -DMOE355_TILED16_T=" in mk
    assert sorted(_tiled16_instances()) == ["bf16_down", "bf16_gate_up", "f16_down", "f16_gate_up"]


def _compile_instance(inst, out):
    dtype, proj = inst.split("_", 1)
    return subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
                           "-Xclang", "-packed-fp32-ops", *_tiled_flags(), f"-DMOE355_TILED16_T={dtype}",
                           f"-DMOE355_TILED16_GATE_UP={'true' if proj == 'gate_up' else 'false'}",
                           "--cuda-device-only", "-S", os.path.join(CSRC, "ffn_tiled16.hip"), "-o", str(out)],
                          capture_output=True, text=True, cwd=CSRC)


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_tiled16_accumulators_stay_in_their_agprs(tmp_path):
    insts = _tiled16_instances()
    outs = [tmp_path / f"ffn_tiled16_{i}.s" for i in insts]
    # the four instances compile in parallel (minutes each)
    with concurrent.futures.ThreadPoolExecutor(len(insts)) as pool:
        results = list(pool.map(_compile_instance, insts, outs))
    for inst, r in zip(insts, results):
        assert r.returncode == 0, f"{inst}: {r.stderr[-2000:]}"
    for asm in outs:
        _check_asm(asm)


def _check_asm(asm):
    lines = asm.read_text().splitlines()
    starts = [i for i, l in enumerate(lines) if re.match(r"^_Z\S*ffn_tiled16_kernel\S*:", l)]
    assert len(starts) == 2, asm  # ragged or not
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
        # The fixed operand fragments v128-v255 are named only by the inline
        # assembly: the kernel's arch VGPR count must still cover them, or
        # the accumulators (AGPRs after accum_offset) would overlap them.
        assert re.search(rf"{re.escape(name)}\.num_vgpr, 256\b", meta), name
        assert re.search(rf"{re.escape(name)}\.private_seg_size, 0\b", meta), name
    offsets = [int(m) for m in re.findall(r"\.amdhsa_accum_offset (\d+)", asm.read_text())]
    assert len(offsets) == 2 and all(o >= 256 for o in offsets), offsets
