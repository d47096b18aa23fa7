"""Builds libllk_gfx950.so (HIP kernels for gfx950 + the C ABI) in-tree.

    python -m dslcompiler_amd.build            # library + tools
    python -m dslcompiler_amd.build --lib-only

Objects go to dslcompiler_amd/_build/, the library to
dslcompiler_amd/libllk_gfx950.so, and the per-operation gfx950 code objects
the kernel cache loads at run time (hipModuleLoadData) to
dslcompiler_amd/objects/.  HIP sources are compiled with
``hipcc --offload-arch=gfx950``; pure C++ runtime sources with g++.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libllk_gfx950.so"
BIN = PKG / "bin"
OBJECTS = PKG / "objects"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX_HOST", "g++")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

# Packed-FP32 VALU forms (v_pk_*_f32) are disabled for all device code: some
# of their forms have given wrong results on MI355X machines of this pool.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function"]
INCLUDES = [f"-I{ROOT / 'include'}", f"-I{CSRC}"]

HIP_SOURCES = [
    CSRC / "kernels" / "mfma_tile.hip",
    CSRC / "kernels" / "swiglu_wide.hip",
    CSRC / "kernels" / "swiglu_decode.hip",
    CSRC / "kernels" / "pack.hip",
    CSRC / "llk_abi.cpp",  # host code that calls the HIP runtime
    CSRC / "kernel_fn.cpp",
    CSRC / "code_object.cpp",
]
# Host sources built by hipcc (they call the HIP runtime or hold device data).
HIP_HOST_SOURCES = {"llk_abi.cpp", "kernel_fn.cpp", "code_object.cpp"}
# One code object per operation (kernels/code_object.hip with LLK_CO_OP),
# named as code_object.cpp looks them up.
CODE_OBJECTS = {"llk_fused_swiglu_gfx950.hsaco": 1, "llk_matmul_gfx950.hsaco": 0}
CXX_SOURCES = [
    CSRC / "runtime" / "json.cpp",
    CSRC / "runtime" / "schedule.cpp",
    CSRC / "runtime" / "packed_layout.cpp",
    CSRC / "runtime" / "tunables.cpp",
    CSRC / "runtime" / "synth.cpp",
    CSRC / "runtime" / "kernel_cache.cpp",
]
TOOLS = {
    "llk-bench": CSRC / "tools" / "llk_bench.cpp",
    "llk-compile": CSRC / "tools" / "llk_compile.cpp",
    "llk-tune": CSRC / "tools" / "llk_tune.cpp",
}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "is not a recognized feature for this target" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _obj(src: Path) -> Path:
    return BUILD / (src.name + ".o")


def _compile(src: Path) -> Path:
    obj = _obj(src)
    if src.suffix == ".hip" or src.name in HIP_HOST_SOURCES:
        cmd = [HIPCC, *HIP_FLAGS, *INCLUDES]
        if src.suffix == ".cpp":
            cmd += ["-x", "hip"]
        cmd += ["-c", str(src), "-o", str(obj)]
    else:
        cmd = [CXX, *CXX_FLAGS, *INCLUDES, "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def _code_object(name: str) -> Path:
    out = OBJECTS / name
    tmp = out.with_suffix(".hsaco.tmp")
    _run([HIPCC, *HIP_FLAGS, *INCLUDES, "--genco", "--no-gpu-bundle-output",
          f"-DLLK_CO_OP={CODE_OBJECTS[name]}", str(CSRC / "kernels" / "code_object.hip"),
          "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build(lib_only: bool = False, jobs: int | None = None) -> Path:
    """Compiles every source, links the library and builds the code objects
    (always a full rebuild)."""
    BUILD.mkdir(exist_ok=True)
    OBJECTS.mkdir(exist_ok=True)
    sources = HIP_SOURCES + [s for s in CXX_SOURCES if s.exists()]
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        cos = [ex.submit(_code_object, n) for n in CODE_OBJECTS]
        objs = list(ex.map(_compile, sources))
        for f in cos:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if not lib_only:
        BIN.mkdir(exist_ok=True)
        for name, src in TOOLS.items():
            if not src.exists():
                continue
            _run([CXX, *CXX_FLAGS, *INCLUDES, str(src), "-o", str(BIN / name),
                  f"-L{PKG}", "-lllk_gfx950", f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,$ORIGIN/..",
                  f"-I{ROCM}/include", "-D__HIP_PLATFORM_AMD__", f"-L{ROCM}/lib", "-lamdhip64",
                  "-pthread"])
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--clean", action="store_true")
    a = ap.parse_args()
    if a.clean and BUILD.exists():
        shutil.rmtree(BUILD)
    print(build(lib_only=a.lib_only, jobs=a.jobs))


if __name__ == "__main__":
    main()
