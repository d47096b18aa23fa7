"""Checks on the gfx950 code objects of the tile kernels, and the small-M
kernel's resource use (CPU only: hipcc cross-compiles the kernel sources to
assembly).

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
# the tile kernel and its row-major form (mfma_tile_rm_kernel: the caller's
# [K, N] weights, A operands by transposed LDS reads); every check below
# holds for both
KERNEL = re.compile(r"^(_ZN10llk_gfx950(?:16mfma_tile_kernel|19mfma_tile_rm_kernel)\w+):", re.M)


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
    assert len([k for k in ks if "16mfma_tile_kernel" in k]) == 12, sorted(ks)
    # row-major: SwiGLU bf16 and fp32 out in both Y forms and split
    # partials; the accumulating GEMM's split partials
    assert sorted(k[len("_ZN10llk_gfx95019mfma_tile_rm_kernelI"):].split("EE")[0]
                  for k in ks if "rm_kernel" in k) == [
        "Li0ELi2ELb1ELb1", "Li1ELi0ELb0ELb0", "Li1ELi0ELb1ELb0", "Li1ELi2ELb0ELb0",
        "Li1ELi2ELb1ELb0", "Li1ELi2ELb1ELb1"], sorted(ks)


def test_k_loop_operand_reads(asm):
    """Per twelve-stage loop body: 96 B-operand reads of 16 bytes; the A
    operands (8 per stage) as 96 more 16-byte reads from the packed payload,
    or, in the row-major form, as 192 transposed 8-byte reads."""
    for name, lines in kernels(asm).items():
        body = [b for b in k_loop(lines) if is_insn(b)]
        b128 = sum(b.startswith("ds_read_b128") for b in body)
        tr = sum(b.startswith("ds_read_b64_tr_b16") for b in body)
        assert (b128, tr) == ((96, 192) if "rm_kernel" in name else (192, 0)), (name, b128, tr)


def test_tile_weight_loads_never_non_temporal(asm):
    """The tile kernel's weight and X loads are ordinary ones in every form:
    its weight panels stream fastest through L2 even when one workgroup reads
    each byte (k-split GEMM M = 200 / 255 and SwiGLU M = 100 measured 6-16%
    slower with `nt`)."""
    for name, lines in kernels(asm).items():
        assert not [b for b in lines if b.startswith("buffer_load") and " nt " in b], name


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


# ---------------------------------------------------------------------------
# The wide SwiGLU tile kernel (kernels/swiglu_wide.hip): the same construction
# with B row blocks per wave (B = 7, 11) -- rows 0-7 accumulate in AGPRs,
# rows 8.. (B = 11) in VGPRs -- and a K-loop body of four 32-k stages whose
# barriers wait for a constant number of loads per stage parity; with and
# without the k split (same K loop, register-order partial stores instead of
# the SiLU epilogue).
# ---------------------------------------------------------------------------
WIDE = re.compile(r"^(_ZN10llk_gfx95023mfma_swiglu_wide_kernelILi(\d+)ELb([01])ELb([01])EE\w+):",
                  re.M)
# loads outstanding at the barriers of an even / odd stage (the refill
# schedule of the kernel's header comment)
WIDE_WAITS = {11: ("13", "11"), 7: ("10", "8")}


@pytest.fixture(scope="module")
def wide_asm(tmp_path_factory) -> str:
    out = tmp_path_factory.mktemp("isa") / "swiglu_wide.s"
    cmd = [B.HIPCC, *B.HIP_FLAGS, *B.INCLUDES, "--cuda-device-only", "-S",
           str(B.CSRC / "kernels" / "swiglu_wide.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def wide_kernels(asm: str) -> dict[tuple[int, int, int], list[str]]:
    """(B, split, non-temporal weights) -> the kernel's instruction lines (as
    kernels())."""
    out = {}
    for m in WIDE.finditer(asm):
        body = asm[m.end():]
        body = body[:body.index("s_endpgm")]
        lines = []
        for ln in body.split("\n"):
            ln = ln.split(";")[0].strip()
            if ln and not ln.startswith(".") or re.match(r"^\.LBB\d+_\d+:", ln):
                lines.append(ln)
        out[(int(m.group(2)), int(m.group(3)), int(m.group(4)))] = lines
    return out


def _acc_regs(mfmas: list[str]) -> tuple[set[int], set[int]]:
    """(AGPRs, VGPRs) used as MFMA accumulators."""
    a, v = set(), set()
    for b in mfmas:
        kind, rs = regs(operands(b)[0])
        (a if kind == "a" else v).update(rs)
    return a, v


def test_wide_instantiations_and_no_scratch(wide_asm):
    assert sorted(wide_kernels(wide_asm)) == [(b, sp, nt) for b in (7, 11) for sp in (0, 1)
                                              for nt in (0, 1)]
    # no spills anywhere in the kernels (the epilogue once spilled AGPRs):
    # the metadata entry of each kernel, its name followed by its scratch size
    meta = re.findall(r"\.name:\s+(_ZN10llk_gfx95023mfma_swiglu_wide_kernel\w+)\n"
                      r"\s+\.private_segment_fixed_size:\s+(\d+)", wide_asm)
    assert len(meta) == 8 and all(size == "0" for _, size in meta), meta
    for count in ("sgpr_spill_count", "vgpr_spill_count"):
        spills = re.findall(r"\." + count + r":\s+(\d+)", wide_asm)
        assert spills and all(n == "0" for n in spills), (count, spills)


def test_wide_k_loop_in_place_mfmas(wide_asm):
    for (Bw, _split, _nt), lines in wide_kernels(wide_asm).items():
        body = [b for b in k_loop(lines) if is_insn(b)]
        mf = [b for b in body if b.startswith(MFMA)]
        assert len(mf) == 4 * 8 * Bw, (Bw, len(mf))
        assert not [b for b in body if b.startswith("v_accvgpr")], Bw
        for b in mf:
            ops = operands(b)
            assert ops[0] == ops[3], (Bw, b)
        a, v = _acc_regs(mf)
        assert len(a) == 4 * 8 * min(Bw, 8), (Bw, len(a))
        assert len(v) == 4 * 8 * max(0, Bw - 8), (Bw, len(v))
        # nothing but the MFMAs writes a VGPR accumulator inside the loop
        for b in body:
            if not b.startswith(MFMA) and operands(b) and not re.match(
                    r"^(ds_write|global_store|buffer_store|buffer_load|s_)", b):
                kind, dst = regs(operands(b)[0])
                assert not (kind == "v" and dst & v), (Bw, b)


def test_wide_k_loop_waits_and_m0(wide_asm):
    for (Bw, _split, _nt), lines in wide_kernels(wide_asm).items():
        body = [b for b in k_loop(lines) if is_insn(b)]
        vm = [re.search(r"vmcnt\((\d+)\)", b).group(1) for b in body if "vmcnt" in b]
        even, odd = WIDE_WAITS[Bw]
        assert sorted(vm) == sorted([even, odd, even, odd]), (Bw, vm)
        assert sum(b == "s_barrier" for b in body) == 4, Bw
        insns = [b for b in lines if is_insn(b)]
        m0 = [k for k, b in enumerate(insns) if "m0" in b]
        assert all(insns[k].startswith("s_mov_b32 m0,") for k in m0), Bw
        dma = [k for k, b in enumerate(insns)
               if b.startswith("buffer_load_dwordx4") and b.endswith(" lds")]
        assert len(dma) == len(m0), Bw
        for a, b in zip(m0, m0[1:] + [len(insns)]):
            loads = [k for k in dma if a < k < b]
            assert len(loads) == 1 and loads[0] >= a + 2, (Bw, insns[a:a + 4])


def test_wide_weight_loads_non_temporal_for_one_m_tile(wide_asm):
    """The WNT forms (one m tile: each weight byte read by one workgroup)
    load every weight stage non-temporal and X as ordinary loads; the other
    forms load nothing non-temporal."""
    for (Bw, split, nt), lines in wide_kernels(wide_asm).items():
        dma = [b for b in lines if b.startswith("buffer_load_dwordx4") and b.endswith(" lds")]
        n_nt = sum(" nt " in b for b in dma)
        if not nt:
            assert n_nt == 0, (Bw, split)
            continue
        # a weight load's resource is the Wg or Wu one, X's is the third
        rsrc = {}
        for b in dma:
            rsrc.setdefault(operands(b)[1], set()).add(" nt " in b)
        assert sorted(map(sorted, rsrc.values())) == [[False], [True], [True]], (Bw, rsrc)


def test_wide_wait_states_around_the_mfmas(wide_asm):
    for (Bw, _split, _nt), lines in wide_kernels(wide_asm).items():
        insns = [b for b in lines if is_insn(b)]
        idx = [k for k, b in enumerate(insns) if b.startswith(MFMA)]
        first, last = idx[0], idx[-1]
        a, v = _acc_regs([insns[k] for k in idx])
        # the last write of an accumulator (zeroing) before the first MFMA
        zero = [k for k, b in enumerate(insns[:first]) if operands(b) and (
            (b.startswith("v_accvgpr_write") and regs(operands(b)[0])[1] & a) or
            (b.startswith("v_") and regs(operands(b)[0])[0] == "v" and regs(operands(b)[0])[1] & v))]
        assert zero, Bw
        assert _nops(insns[zero[-1]:first]) >= 64, (Bw, "zeroing -> first MFMA")
        # the first read of an accumulator after the last MFMA
        def reads_acc(b):
            if b.startswith(MFMA) or not operands(b):
                return False
            ops = operands(b)
            srcs = ops if re.match(r"^(ds_write|global_store|buffer_store|flat_store)", b) else ops[1:]
            return any((regs(o)[0] == "a" and regs(o)[1] & a) or (regs(o)[0] == "v" and regs(o)[1] & v)
                       for o in srcs)
        reads = [k for k, b in enumerate(insns) if k > last and reads_acc(b)]
        assert reads, Bw
        assert _nops(insns[last:reads[0]]) >= 64, (Bw, "last MFMA -> first read")


def test_wide_no_valu_writes_mfma_operands_just_before(wide_asm):
    for (Bw, _split, _nt), lines in wide_kernels(wide_asm).items():
        insns = [b for b in lines if is_insn(b)]
        for k, b in enumerate(insns):
            if not b.startswith(MFMA):
                continue
            ops = operands(b)
            src = regs(ops[1])[1] | regs(ops[2])[1]
            for prev in insns[max(0, k - 4):k]:
                if prev.startswith("v_") and not prev.startswith("v_mfma"):
                    kind, dst = regs(operands(prev)[0]) if operands(prev) else ("", set())
                    assert not (kind == "v" and dst & src), (Bw, prev, b)


# ---- small-M kernel ---------------------------------------------------------

@pytest.fixture(scope="module")
def skinny_asm(tmp_path_factory) -> str:
    out = tmp_path_factory.mktemp("isa") / "swiglu_decode.s"
    cmd = [B.HIPCC, *B.HIP_FLAGS, *B.INCLUDES, "--cuda-device-only", "-S",
           str(B.CSRC / "kernels" / "swiglu_decode.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def test_small_m_kernels_no_scratch_and_pipelined_forms(skinny_asm):
    """Every small-M instantiation with vector X loads runs without scratch
    (the pipelined loop holds two 64-k steps of weights in registers); the
    element-wise X forms (unaligned X rows) of the 16-wave SwiGLU shapes keep
    one 8-byte spill, stored before the K loop and reloaded after it, within
    12 bytes of scratch.  The SwiGLU form for M > 32 (two 32-row tiles, one
    wave group of two column groups, four waves) with vector X loads is the
    pipelined one, the GEMM's is not."""
    meta = dict(re.findall(r"\.name:\s+(_ZN10llk_gfx95013skinny_kernel\w+)\n"
                           r"\s+\.private_segment_fixed_size:\s+(\d+)", skinny_asm))
    assert len(meta) >= 24, sorted(meta)
    # NMAT, MT, KS, G, GW, OUT, XVEC, UNROLL, PIPE
    sym = re.compile(r"skinny_kernelILi(\d)ELi(\d)ELi(\d+)ELi(\d)ELi(\d)ELi(\d)ELb(\d)ELi(\d)ELb(\d)E")
    forms = [tuple(int(v) for v in sym.search(name).groups()) for name in meta]
    for f, size in zip(forms, meta.values()):
        if f[6] == 1:
            assert size == "0", (f, size)
        else:
            assert int(size) <= 12 and (size == "0" or f[2] * f[3] == 16), (f, size)
    swiglu_m64 = [f for f in forms if f[:5] == (2, 2, 4, 1, 2) and f[6] == 1]
    gemm_m64 = [f for f in forms if f[:5] == (1, 2, 4, 1, 2) and f[6] == 1]
    assert swiglu_m64 and all(f[8] == 1 for f in swiglu_m64), swiglu_m64
    assert gemm_m64 and all(f[8] == 0 for f in gemm_m64), gemm_m64


def test_decode_tile_kernel_loop(skinny_asm):
    """The decode tile kernel (every instantiation: MT = 1, 2, 4 32-row MFMA
    tiles per wave on the packed payload, MT = 1, 2 on row-major weights):
    no scratch; its K loop (one 64-k step; the loop region with the barrier)
    holds exactly one vector-memory wait, vmcnt(4 + 2 MT) -- the wave's loads
    of the next step may still be in flight -- then one barrier, four
    non-temporal weight LDS-DMA loads and 2 MT X ones, each right after its
    own M0 write and one wait state, and 8 MT v_mfma_f32_32x32x16_bf16; the
    packed forms read each A operand as one 16-byte LDS load, the row-major
    ones as two transposed 8-byte reads (16 ds_read_b64_tr_b16 per step)."""
    names = re.findall(r"^(_ZN10llk_gfx95018decode_tile_kernel\w+):", skinny_asm, re.M)
    form = r"decode_tile_kernelILi\d+ELi\d+ELi(\d+)ELb(\d)E"
    # (SwiGLU bf16 / fp32, GEMM bf16 / fp16 / fp32) x (MT 1, 2, 4 packed; 1, 2 row-major)
    assert len(names) == 25, names
    forms = sorted((int(re.search(form, n).group(1)), int(re.search(form, n).group(2)))
                   for n in names)
    assert forms == sorted([(mt, 0) for mt in (1, 2, 4)] * 5 + [(mt, 1) for mt in (1, 2)] * 5), forms
    meta = dict(re.findall(r"\.name:\s+(_ZN10llk_gfx95018decode_tile_kernel\w+)\n"
                           r"\s+\.private_segment_fixed_size:\s+(\d+)", skinny_asm))
    assert sorted(meta) == sorted(names) and set(meta.values()) == {"0"}, meta
    for name in names:
        body = skinny_asm[skinny_asm.index(name + ":"):]
        body = body[:body.index("s_endpgm")]
        lines = [ln.split(";")[0].strip() for ln in body.split("\n")]
        lines = [ln for ln in lines if ln]
        labels = {ln[:-1]: i for i, ln in enumerate(lines) if ln.endswith(":")}
        # loop regions: a header label to the last backward branch to it (the
        # conditional X loads give the body more than one path back)
        ends: dict[int, int] = {}
        for i, ln in enumerate(lines):
            m = re.match(r"^s_(?:cbranch_\w+|branch)\s+(\.LBB\d+_\d+)$", ln)
            if m and m.group(1) in labels and labels[m.group(1)] < i:
                ends[labels[m.group(1)]] = i
        loop = [lines[h:e + 1] for h, e in ends.items()
                if any("v_mfma" in b for b in lines[h:e + 1])
                and any(b == "s_barrier" for b in lines[h:e + 1])]
        assert len(loop) == 1, name
        loop = loop[0]
        mt, rm = (int(v) for v in re.search(form, name).groups())
        assert sum("v_mfma_f32_32x32x16_bf16" in b for b in loop) == 8 * mt, name
        tr = sum(b.startswith("ds_read_b64_tr_b16") for b in loop)
        assert tr == (16 if rm else 0), (name, tr)
        assert not any(b.startswith("ds_read_u16") for b in loop), name
        vm = [re.search(r"vmcnt\((\d+)\)", b).group(1) for b in loop
              if b.startswith("s_waitcnt") and "vmcnt" in b]
        assert vm == [str(4 + 2 * mt)], (name, vm)
        assert sum(b == "s_barrier" for b in loop) == 1, name
        loads = [i for i, b in enumerate(loop) if b.startswith("buffer_load") and b.endswith("lds")]
        assert len(loads) == 4 + 2 * mt, name
        assert sum(" nt lds" in loop[i] for i in loads) == 4, name
        for i in loads:
            assert loop[i - 2].startswith("s_mov_b32 m0,") and loop[i - 1] == "s_nop 0", \
                (name, loop[i - 2:i + 1])
        assert sum(b.startswith("s_mov_b32 m0,") for b in loop) == 4 + 2 * mt, name
