"""The object-code level's gfx950 code objects on the host: one per
operation, built beside the library; each is read and checked before any
HIP call (a 64-bit AMDGPU ELF for gfx950 with kernels), and a missing or
wrong object is a status from lookupOrCompile, with nothing cached (the
reference's lookupOrCompile returns an error instead of an entry when
lowering or symbol lookup fails: JitCache.cpp:182-245).  Loading and running
an entry is tests/test_gpu_code_object.py."""
from __future__ import annotations

import re
import shutil
import struct
from pathlib import Path

import pytest

import dslcompiler_amd as llk
from dslcompiler_amd import cache
from dslcompiler_amd.cache import JitCache, KernelKey

PKG = Path(llk.__file__).resolve().parent
TILE = "_ZN10llk_gfx95016mfma_tile_kernelI"
# the 128-column SwiGLU tiles: mfma_tile_kernel<1, 0, true, false>(TileArgs)
CONFIG3 = TILE + "Li1ELi0ELb1ELb0EEEvNS_8TileArgsE"


def _key(op, out=0):
    return KernelKey(operation=op, isa=7, N=128, K=64, output_type=out)


def test_default_paths_are_beside_the_library():
    for op, name in ((cache.OP_FUSED_SWIGLU, "llk_fused_swiglu_gfx950.hsaco"),
                     (cache.OP_MATMUL, "llk_matmul_gfx950.hsaco")):
        p = Path(cache.code_object_path(op))
        assert p == PKG / "objects" / name and p.is_file()
        assert cache.code_object_path(op, "/some/dir") == f"/some/dir/{name}"
    with pytest.raises(llk.LLKError, match="INVALID_ARGUMENT"):
        cache.code_object_path(1)  # RoPE: no code object


def test_objects_hold_their_operations_kernels():
    sw = cache.code_object_info(cache.code_object_path(cache.OP_FUSED_SWIGLU))
    mm = cache.code_object_info(cache.code_object_path(cache.OP_MATMUL))
    assert CONFIG3 in sw and CONFIG3 not in mm
    # tile kernels: MODE 1 only in the SwiGLU object, MODE 0 only in the GEMM one
    assert {k[len(TILE):len(TILE) + 4] for k in sw if k.startswith(TILE)} == {"Li1E"}
    assert {k[len(TILE):len(TILE) + 4] for k in mm if k.startswith(TILE)} == {"Li0E"}
    # both operations' launchers: tile (5 / 7 instantiations), k-split
    # reduce, wide SwiGLU tiles (2 widths x split x non-temporal weights),
    # small-M kernels (2 x 3 widths x 2 X paths x output types) and their
    # reduce, decode tile kernels (output types x 64-, 128- and 256-row
    # forms on the packed payload, 64- and 128-row forms on row-major
    # weights), X padding and the K = 0
    # fill; no tile form waits for another workgroup (every instantiation has
    # the four template arguments MODE, OUT, YVEC, SPLIT)
    def count(names, part):
        return sum(part in k for k in names)
    assert (count(sw, "mfma_tile_kernel"), count(mm, "mfma_tile_kernel")) == (5, 7)
    for k in sw + mm:
        if k.startswith(TILE):
            args = k[len(TILE):k.index("EEvNS_8TileArgsE")]
            assert len(re.findall(r"L[ib]\d+E", args)) == 4, k
    assert (count(sw, "mfma_swiglu_wide_kernel"), count(mm, "mfma_swiglu_wide_kernel")) == (8, 0)
    assert (count(sw, "13skinny_kernel"), count(mm, "13skinny_kernel")) == (24, 36)
    assert (count(sw, "decode_tile_kernel"), count(mm, "decode_tile_kernel")) == (10, 15)
    for names in (sw, mm):
        assert "_Z15pad_rows_kernelPKtliiPtl" in names
        assert "_Z16zero_rows_kernelPhllil" in names
        assert "_ZN10llk_gfx95016pack_tile_kernelEPKtliiiiPj" in names  # KernelFn entries pack


def _expect(path_or_dir, key, match):
    c = JitCache()
    c.set_object_dir(str(path_or_dir))
    with pytest.raises(llk.LLKError, match=match):
        c.lookup_or_compile(key)
    assert c.lookup_object_code(key) is None and c.size() == 0
    c.close()


def test_missing_object_is_a_status(tmp_path):
    _expect(tmp_path, _key(cache.OP_FUSED_SWIGLU), "NOT_FOUND.*llk_fused_swiglu_gfx950.hsaco")
    _expect(tmp_path / "absent", _key(cache.OP_MATMUL), "NOT_FOUND.*llk_matmul_gfx950.hsaco")


def test_object_for_another_gpu_is_rejected(tmp_path):
    src = Path(cache.code_object_path(cache.OP_FUSED_SWIGLU))
    data = bytearray(src.read_bytes())
    # e_flags (offset 48): the low byte is the AMDGPU machine; 0x4c = gfx942
    (flags,) = struct.unpack_from("<I", data, 48)
    assert flags & 0xFF == 0x4F
    struct.pack_into("<I", data, 48, (flags & ~0xFF) | 0x4C)
    bad = tmp_path / src.name
    bad.write_bytes(bytes(data))
    with pytest.raises(llk.LLKError, match="UNSUPPORTED_ARCH.*0x4c, not gfx950"):
        cache.code_object_info(str(bad))
    _expect(tmp_path, _key(cache.OP_FUSED_SWIGLU), "UNSUPPORTED_ARCH")


def test_host_elf_and_junk_are_rejected(tmp_path):
    host = tmp_path / "host"
    host.mkdir()
    shutil.copy(PKG / "libllk_gfx950.so", host / "llk_matmul_gfx950.hsaco")  # an x86-64 ELF
    _expect(host, _key(cache.OP_MATMUL), "UNSUPPORTED_ARCH.*not AMDGPU")
    junk = tmp_path / "junk"
    junk.mkdir()
    (junk / "llk_matmul_gfx950.hsaco").write_text("not a code object\n" * 8)
    _expect(junk, _key(cache.OP_MATMUL), "INVALID_ARGUMENT.*not a 64-bit")
    cut = tmp_path / "cut"
    cut.mkdir()
    src = Path(cache.code_object_path(cache.OP_MATMUL)).read_bytes()
    (cut / "llk_matmul_gfx950.hsaco").write_bytes(src[:200])
    _expect(cut, _key(cache.OP_MATMUL), "INVALID_ARGUMENT.*malformed section headers")


def test_entries_are_bound_per_output_type():
    c = JitCache()
    bf16 = c.lookup_or_compile(_key(cache.OP_MATMUL, 0)).address
    f32 = c.lookup_or_compile(_key(cache.OP_MATMUL, 2)).address
    sw = c.lookup_or_compile(_key(cache.OP_FUSED_SWIGLU, 0)).address
    assert len({bf16, f32, sw}) == 3
    assert c.lookup_or_compile(_key(cache.OP_MATMUL, 2)).address == f32
    c.close()
