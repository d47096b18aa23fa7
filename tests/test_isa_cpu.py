"""Checks on the gfx950 code object of the tile kernel (CPU only: hipcc
cross-compiles the kernel source to assembly).

The tile kernel issues its v_mfma_f32_16x16x32_bf16 instructions from inline
assembly with the accumulators tied to AGPRs, so the compiler's hazard
recognizer does not see them.  The kernel keeps the hazards away by
construction; these tests hold that construction on the instructions the
compiler actually emitted, for every instantiation:

* the K loop body (twelve 32-k stages: the period of the two LDS rings, so
  every ring slot is a compile-time constant) is exactly 768 MFMAs with no
  AGPR copies (the reason for the inline assembly) and every MFMA
  accumulates in place;
* its only vector-memory waits are the twelve barriers' (16 loads
  outstanding each: the refills are spread evenly; the LDS-DMA loads are
  inline assembly too, so that the compiler adds no waits of its own), and M0
  is written only by the loads' own s_mov, each followed by exactly one
  LDS-DMA load with at least one instruction (the wait state) between them;
* no VALU instruction writes an MFMA's A/B operand registers shortly before
  it (operands must come from LDS loads, whose waits the compiler places);
* nothing writes an AGPR between the MFMAs except the MFMAs themselves;
* at least 64 wait states (four `s_nop 15`) separate the accumulators'
  zeroing from the first MFMA and the last MFMA from the first accumulator
  read.
"""
from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

from dslcompiler_amd import build as B  # noqa: E402

MFMA = "v_mfma_f32_16x16x32_bf16"
KERNEL = re.compile(r"^(_ZN10llk_gfx95016mfma_tile_kernel\w+):", re.M)


@pytest.fixture(scope="module")
def asm(tmp_path_factory) -> str:
    out = tmp_path_factory.mktemp("isa") / "mfma_tile.s"
    cmd = [B.HIPCC, *B.HIP_FLAGS, *B.INCLUDES, "--cuda-device-only", "-S",
           str(B.CSRC / "kernels" / "mfma_tile.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def kernels(asm: str) -> dict[str, list[str]]:
    """Kernel name -> its instruction lines (labels kept, comments dropped)."""
    out = {}
    for m in KERNEL.finditer(asm):
        body = asm[m.end():]
        body = body[:body.index("s_endpgm")]
        lines = []
        for ln in body.split("\n"):
            ln = ln.split(";")[0].strip()
            if ln and not ln.startswith(".") or re.match(r"^\.LBB\d+_\d+:", ln):
                lines.append(ln)
        out[m.group(1)] = lines
    return out


def regs(tok: str) -> tuple[str, set[int]]:
    """'v[4:7]' -> ('v', {4,5,6,7}); 'a12' -> ('a', {12}); else ('', set())."""
    tok = tok.strip().rstrip(",")
    m = re.match(r"^([va])\[(\d+):(\d+)\]$", tok)
    if m:
        return m.group(1), set(range(int(m.group(2)), int(m.group(3)) + 1))
    m = re.match(r"^([va])(\d+)$", tok)
    if m:
        return m.group(1), {int(m.group(2))}
    return "", set()


def operands(line: str) -> list[str]:
    """Register/immediate operands in order (modifiers such as offset:16 dropped)."""
    parts = line.split(None, 1)
    return [t.strip().split()[0] for t in parts[1].split(",") if t.strip()] if len(parts) > 1 else []


def reads_agpr(line: str) -> bool:
    """Whether a non-MFMA instruction reads an AGPR (v_accvgpr_read, or a
    store / LDS write taking AGPR data)."""
    ops = operands(line)
    srcs = ops[1:] if not re.match(r"^(ds_write|global_store|buffer_store|flat_store)", line) else ops
    return any(regs(o)[0] == "a" for o in srcs)


def is_insn(line: str) -> bool:
    return not line.endswith(":")


def k_loop(lines: list[str]) -> list[str]:
    """The innermost backward-branching region that contains MFMAs."""
    labels = {ln[:-1]: i for i, ln in enumerate(lines) if ln.endswith(":")}
    best = None
    for i, ln in enumerate(lines):
        m = re.match(r"^s_cbranch_\w+\s+(\.LBB\d+_\d+)$", ln)
        if m and m.group(1) in labels and labels[m.group(1)] < i:
            body = lines[labels[m.group(1)]:i + 1]
            if any(MFMA in b for b in body) and (best is None or len(body) < len(best)):
                best = body
    assert best is not None, "no K loop found"
    return best


def test_every_tile_instantiation_found(asm):
    ks = kernels(asm)
    # SwiGLU (bf16/fp32 out, both Y vector forms, split partials) and GEMM
    # (bf16/fp16/fp32 out, both forms, split partials)
    assert len(ks) >= 10, sorted(ks)


def test_k_loop_is_768_in_place_mfmas_without_agpr_copies(asm):
    for name, lines in kernels(asm).items():
        body = [b for b in k_loop(lines) if is_insn(b)]
        mf = [b for b in body if b.startswith(MFMA)]
        assert len(mf) == 12 * 64, (name, len(mf))
        assert not [b for b in body if b.startswith("v_accvgpr")], name
        for b in mf:
            ops = operands(b)
            assert ops[0] == ops[3] and ops[0].startswith("a["), (name, b)


def test_k_loop_waits_and_m0(asm):
    for name, lines in kernels(asm).items():
        body = [b for b in k_loop(lines) if is_insn(b)]
        vm = [b for b in body if "vmcnt" in b]
        assert [re.search(r"vmcnt\((\d+)\)", b).group(1) for b in vm] == ["16"] * 12, (name, vm)
        assert sum(b == "s_barrier" for b in body) == 12, name
        insns = [b for b in lines if is_insn(b)]
        m0 = [k for k, b in enumerate(insns) if "m0" in b]
        assert all(insns[k].startswith("s_mov_b32 m0,") for k in m0), name
        dma = [k for k, b in enumerate(insns)
               if b.startswith("buffer_load_dwordx4") and b.endswith(" lds")]
        assert len(dma) == len(m0), name
        for a, b in zip(m0, m0[1:] + [len(insns)]):
            loads = [k for k in dma if a < k < b]
            assert len(loads) == 1 and loads[0] >= a + 2, (name, insns[a:a + 4])


def test_no_valu_writes_mfma_operands_just_before(asm):
    for name, lines in kernels(asm).items():
        insns = [b for b in lines if is_insn(b)]
        for k, b in enumerate(insns):
            if not b.startswith(MFMA):
                continue
            ops = operands(b)
            src = regs(ops[1])[1] | regs(ops[2])[1]
            for prev in insns[max(0, k - 4):k]:
                if prev.startswith("v_") and not prev.startswith("v_mfma"):
                    kind, dst = regs(operands(prev)[0]) if operands(prev) else ("", set())
                    assert not (kind == "v" and dst & src), (name, prev, b)


def test_agprs_written_only_by_mfmas_between_first_and_last_mfma(asm):
    for name, lines in kernels(asm).items():
        insns = [b for b in lines if is_insn(b)]
        idx = [k for k, b in enumerate(insns) if b.startswith(MFMA)]
        for b in insns[idx[0]:idx[-1] + 1]:
            store = re.match(r"^(ds_write|global_store|buffer_store|flat_store|s_)", b)
            if not b.startswith(MFMA) and not store and operands(b):
                assert regs(operands(b)[0])[0] != "a", (name, b)


def _nops(seq: list[str]) -> int:
    return sum(int(b.split()[1]) + 1 for b in seq if b.startswith("s_nop"))


def test_wait_states_around_the_mfmas(asm):
    for name, lines in kernels(asm).items():
        insns = [b for b in lines if is_insn(b)]
        idx = [k for k, b in enumerate(insns) if b.startswith(MFMA)]
        first, last = idx[0], idx[-1]
        writes = [k for k, b in enumerate(insns[:first]) if b.startswith("v_accvgpr_write")]
        assert writes, name
        assert _nops(insns[writes[-1]:first]) >= 64, (name, "zeroing -> first MFMA")
        reads = [k for k, b in enumerate(insns)
                 if k > last and not b.startswith(MFMA) and reads_agpr(b)]
        assert reads, name
        assert _nops(insns[last:reads[0]]) >= 64, (name, "last MFMA -> first read")
