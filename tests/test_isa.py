"""Checks on the gfx950 assembly of the attention kernels (no GPU needed; hipcc cross-compiles).

Every LDS DMA that takes its global base from SGPRs (global_load_lds_dwordx4 vOFF, s[a:b]) must read
SGPRs that an SALU instruction wrote immediately before it.  When the compiler keeps the base in
VGPRs, it forms the SGPR pair with v_readfirstlane, a VALU write; a VMEM instruction that reads SGPRs
needs 5 wait states after a VALU write of them, and the compiler does not insert them across inline
asm.  A build in which the DMA read v_readfirstlane results one to three instructions later faulted
the GPU (the base's low half was stale).  dma16s copies the base with s_mov_b64 inside its asm, and
this test pins that every such DMA in the built kernels goes through the copy."""

import os
import re
import shutil
import subprocess
import tempfile

import pytest

from pe_ablations_amd import build as B

DMA_SOURCES = ["pe_fwd.hip", "pe_bwd.hip", "pe_decode.hip"]


def device_asm(src: str, out_dir: str) -> subprocess.Popen:
    out = os.path.join(out_dir, os.path.splitext(src)[0] + ".s")
    cmd = [B.hipcc()] + B.common_flags() + ["-x", "hip", "--cuda-device-only", "-S",
                                            os.path.join(B.CSRC, src), "-o", out]
    return subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, text=True), out


@pytest.fixture(scope="module")
def asm_texts():
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc is not available")
    with tempfile.TemporaryDirectory() as d:
        jobs = [device_asm(s, d) for s in DMA_SOURCES]
        texts = {}
        for (p, out), src in zip(jobs, DMA_SOURCES):
            _, err = p.communicate(timeout=600)
            assert p.returncode == 0, err[-2000:]
            texts[src] = open(out).read()
    return texts


def instructions(text):
    for line in text.split("\n"):
        t = line.strip()
        if not t or t.startswith((";", ".", "//")) or t.endswith(":"):
            continue
        yield t


def test_sgpr_based_lds_dma_reads_an_salu_copy(asm_texts):
    n = 0
    for src, text in asm_texts.items():
        prev = None
        for ins in instructions(text):
            m = re.match(r"global_load_lds_dwordx4\s+v\d+,\s*(s\[\d+:\d+\])", ins)
            if m:
                n += 1
                assert prev is not None and re.match(r"s_mov_b64\s+" + re.escape(m.group(1)) + r",", prev), \
                    f"{src}: SGPR-based LDS DMA not preceded by an SALU copy of its base: {prev!r} -> {ins!r}"
            prev = ins
    assert n > 0, "no SGPR-based LDS DMA found: the kernels changed, revisit this check"


def sgprs(operand):
    """The SGPRs an operand names (s7, s[4:5]); empty for anything else."""
    if re.fullmatch(r"s\d+", operand):
        return {operand}
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", operand)
    return {f"s{i}" for i in range(int(m.group(1)), int(m.group(2)) + 1)} if m else set()


def test_no_vmem_reads_a_valu_written_sgpr_within_five_wait_states(asm_texts):
    """The general rule, over every SGPR-addressed global access of the two sources."""
    for src, text in asm_texts.items():
        recent = []  # (SGPRs last written by a VALU instruction, wait states since)
        for ins in instructions(text):
            parts = ins.split(None, 1)
            op = parts[0]
            m = re.match(r"global_\w+\s+.*?(s\[\d+:\d+\])", ins)
            if m:
                regs = sgprs(m.group(1))
                for written, ws in recent:
                    assert not (written & regs), \
                        f"{src}: {ins!r} reads {sorted(written & regs)} {ws} wait states after a VALU write"
            ws_add = int(parts[1]) + 1 if op == "s_nop" else 1
            recent = [(w, ws + ws_add) for w, ws in recent if ws + ws_add < 5]
            dst = sgprs(parts[1].split(",")[0].strip()) if len(parts) > 1 else set()
            if op.startswith("v_") and dst:
                recent.append((dst, 0))
            elif op.startswith("s_") and dst:
                recent = [(w - dst, ws) for w, ws in recent if w - dst]
