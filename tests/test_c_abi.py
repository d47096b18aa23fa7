"""The C ABI from plain C: tests/c_abi/host_only.c is compiled as C99 with
-Wall -Wextra -pedantic -Werror against include/llk/llk_abi.h, linked to the
library, and run (host-only calls; no GPU)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIBDIR = ROOT / "dslcompiler_amd"


def test_header_and_library_from_c(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    assert (LIBDIR / "libllk_gfx950.so").exists(), "library not built"
    exe = tmp_path / "host_only"
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror",
           f"-I{ROOT / 'include'}", str(Path(__file__).parent / "c_abi" / "host_only.c"),
           "-o", str(exe), f"-L{LIBDIR}", "-lllk_gfx950", f"-Wl,-rpath,{LIBDIR}"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c abi ok" in r.stdout
