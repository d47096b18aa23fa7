"""Writes tests/golden/ref_vectors.npz and tests/golden/config1_samples.npz.

ref_vectors.npz -- the reference's own SwiGLU test cases:
  * inputs reproduced bit for bit the way the reference tests draw them
    (tests/golden/ref_inputs.cpp: libstdc++ mt19937(42) +
    normal_distribution<float>, the tests' f32->bf16 helper);
  * expected outputs computed by the reference's OWN routines, compiled from
    its sources into oracle/_ref/libref.so:
      swiglu_reference_fp64  (test/Execution/swiglu_reference.cpp:77-99)
      swiglu_reference       (test/Execution/swiglu_reference.cpp:38-70, fp32)
  Shapes [M, N, K]: swiglu_vector_avx2.cpp:214-218 and swiglu_scalar.cpp:355
  ("vec", bf16 inputs) and swiglu_reference.cpp:109-113 ("ref", fp32 inputs).

config1_samples.npz -- BASELINE config 1 (M=64, K=512, N=1376, seed 42 of
the library's generator): 512 sampled output positions with the CPU oracle's
fp32 and bf16 values (a regression pin for both the oracle and the kernels).

Needs /root/reference (for oracle/_ref) and g++; run from the repo root:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

VEC_SHAPES = [(32, 128, 256), (16, 512, 512), (32, 256, 127), (4, 8, 3)]
REF_SHAPES = [(1, 4, 2), (2, 3, 4), (4, 8, 16)]


def _reproducer(tmp: Path) -> Path:
    exe = tmp / "ref_inputs"
    subprocess.run(["g++", "-O2", "-std=c++17", str(HERE / "ref_inputs.cpp"), "-o", str(exe)],
                   check=True)
    return exe


def _draw(exe: Path, mode: str, M: int, N: int, K: int, dtype) -> tuple:
    raw = subprocess.run([str(exe), mode, str(M), str(N), str(K)], check=True,
                         stdout=subprocess.PIPE).stdout
    a = np.frombuffer(raw, dtype=dtype)
    x = a[:M * K].reshape(M, K)
    wg = a[M * K:M * K + K * N].reshape(K, N)
    wu = a[M * K + K * N:].reshape(K, N)
    return x.copy(), wg.copy(), wu.copy()


def main() -> None:
    import oracle
    from common import bf16_bits_to_f32
    ref = oracle.ref()
    if ref is None:
        oracle.build(ref=True)
        ref = oracle.ref()
    if ref is None:
        raise SystemExit("oracle/_ref is not built (needs the reference tree)")
    out = {}
    with tempfile.TemporaryDirectory() as td:
        exe = _reproducer(Path(td))
        for (M, N, K) in VEC_SHAPES:
            x, wg, wu = _draw(exe, "vec", M, N, K, np.uint16)
            xd, gd, ud = (bf16_bits_to_f32(a).astype(np.float64) for a in (x, wg, wu))
            y64 = np.empty((M, N), np.float64)
            ref.ref_swiglu_fp64(np.ascontiguousarray(xd), np.ascontiguousarray(gd),
                                np.ascontiguousarray(ud), y64, M, N, K)
            tag = f"vec_M{M}_N{N}_K{K}"
            out[tag + "_x"], out[tag + "_wg"], out[tag + "_wu"] = x, wg, wu
            out[tag + "_y_fp64"] = y64
        for (M, N, K) in REF_SHAPES:
            x, wg, wu = _draw(exe, "ref", M, N, K, np.float32)
            y32 = np.empty((M, N), np.float32)
            ref.ref_swiglu_fp32(x, wg, wu, y32, M, N, K)
            y64 = np.empty((M, N), np.float64)
            ref.ref_swiglu_fp64(x.astype(np.float64), wg.astype(np.float64),
                                wu.astype(np.float64), y64, M, N, K)
            tag = f"ref_M{M}_N{N}_K{K}"
            out[tag + "_x"], out[tag + "_wg"], out[tag + "_wu"] = x, wg, wu
            out[tag + "_y_fp32"], out[tag + "_y_fp64"] = y32, y64
    np.savez_compressed(HERE / "ref_vectors.npz", **out)

    # BASELINE config 1 samples from the CPU oracle.
    from common import swiglu_inputs
    x, wg, wu = swiglu_inputs(64, 512, 1376, seed=42)
    yf, yb = oracle.swiglu(x, wg, wu)
    rng = np.random.default_rng(1234)
    idx = rng.choice(64 * 1376, size=512, replace=False)
    np.savez_compressed(HERE / "config1_samples.npz", index=idx.astype(np.int64),
                        y_fp32=yf.ravel()[idx], y_bf16=yb.ravel()[idx],
                        x_checksum=np.array([int(x.astype(np.uint64).sum())], np.uint64),
                        w_checksum=np.array([int(wg.astype(np.uint64).sum() +
                                                 wu.astype(np.uint64).sum())], np.uint64))
    print("wrote", HERE / "ref_vectors.npz", "and", HERE / "config1_samples.npz")


if __name__ == "__main__":
    main()
