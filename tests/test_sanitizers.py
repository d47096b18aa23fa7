"""Host-code sanitizers (CPU only): ThreadSanitizer over the cache's LRU
levels and the oracle's tile pool, AddressSanitizer + UBSan over the host
packers, the JSON parser and the schedule loader, and both over the L4
level's single-flight get-or-pack and counted references.  Built with g++
from the sources (no device code involved)."""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SAN = Path(__file__).resolve().parent / "sanitize"
CSRC = ROOT / "dslcompiler_amd" / "csrc"
RUNTIME = CSRC / "runtime"


def _build_and_run(tmp_path, name, sources, flags, args=()):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path / name
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", *flags,
           f"-I{CSRC}", f"-I{ROOT / 'include'}", "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__",
           *map(str, sources), "-o", str(exe), "-pthread"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if r.returncode != 0 and "sanitize" in r.stderr and "unrecognized" in r.stderr:
        pytest.skip("compiler lacks the sanitizer runtime")
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1", ASAN_OPTIONS="halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", TMPDIR=str(tmp_path))
    r = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Sanitizer" not in r.stderr, r.stderr
    return r.stdout


def test_tsan_lru_levels(tmp_path):
    out = _build_and_run(tmp_path, "lru_race", [SAN / "lru_race.cpp"], ["-fsanitize=thread"])
    assert "lru_race ok" in out


def test_tsan_oracle_tile_pool(tmp_path):
    out = _build_and_run(tmp_path, "pool_race", [SAN / "pool_race.cpp", ROOT / "oracle" / "oracle.cpp"],
                         ["-fsanitize=thread", "-std=c++20"])
    assert "pool_race ok" in out


def test_asan_ubsan_host_runtime(tmp_path):
    db = ROOT / "dslcompiler_amd" / "schedules" / "gfx950" / "schedule_db.json"
    out = _build_and_run(tmp_path, "host_asan",
                         [SAN / "host_asan.cpp", RUNTIME / "packed_layout.cpp",
                          RUNTIME / "json.cpp", RUNTIME / "schedule.cpp"],
                         ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"], [str(db)])
    assert "host_asan ok" in out


@pytest.mark.parametrize("san", ["address,undefined", "thread"])
def test_l4_single_flight_and_counted_references(tmp_path, san):
    """8 threads missing on one key see exactly one pack and one handle;
    acquired handles stay readable while another thread clears and evicts
    the level (a freed handle in use would be a sanitizer report)."""
    out = _build_and_run(tmp_path, "l4_single_flight",
                         [SAN / "l4_single_flight.cpp", RUNTIME / "kernel_cache.cpp",
                          RUNTIME / "packed_layout.cpp"],
                         [f"-fsanitize={san}", "-fno-sanitize-recover=all"])
    assert "l4_single_flight ok:" in out
