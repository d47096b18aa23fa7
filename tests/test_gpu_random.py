"""Seeded randomized parity: 48 configurations drawn from a fixed seed cover
SwiGLU and GEMM over ragged M, N, K (both kernels), every output type, padded
and unpadded X strides, and forced or automatic k splits and group widths.
Each is checked against the oracle to the north-star bar, and the 16-bit
outputs against the rounding of the same kernel's fp32 result."""
from __future__ import annotations

import numpy as np
import pytest

from common import assert_parity, normal_bf16, to_bf16_bits
from gpu_util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _cases(n=48, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        op = "swiglu" if rng.random() < 0.6 else "gemm"
        M = int(rng.choice([rng.integers(1, 65), rng.integers(65, 700)]))
        K = int(rng.integers(1, 1600))
        N = int(rng.integers(1, 1300))
        if M * N * K > 2.5e8:
            continue
        out.append(dict(op=op, M=M, K=K, N=N, pad=int(rng.integers(0, 2)) * int(rng.integers(1, 40)),
                        splits=int(rng.choice([0, 0, 2, 3, 5])), group=int(rng.choice([1, 2, 4])),
                        out=str(rng.choice(["bf16", "f32"] + (["f16"] if op == "gemm" else []))),
                        seed=int(rng.integers(0, 1 << 30))))
    return out


CASES = _cases()


class _Knobs:
    def __init__(self, llk, **kv):
        self.llk, self.kv, self.old = llk, kv, {}

    def __enter__(self):
        for k, v in self.kv.items():
            self.old[k] = self.llk.get_tunable(k)
            self.llk.set_tunable(k, v)

    def __exit__(self, *exc):
        for k, v in self.old.items():
            self.llk.set_tunable(k, v)


@pytest.mark.parametrize("i", range(len(CASES)))
def test_random_configuration(llk, gpu, orc, i):
    c = CASES[i]
    print(f"case random {i}: {c}", flush=True)
    M, K, N = c["M"], c["K"], c["N"]
    s = 1.0 / np.sqrt(K)
    x = normal_bf16(c["seed"], 0, (M, K))
    w0 = normal_bf16(c["seed"], 1, (K, N), s)
    w1 = normal_bf16(c["seed"], 2, (K, N), s)
    xd = to_dev(gpu, x, stride0=K + c["pad"] if c["pad"] else None)
    p0 = llk.PackedWeights.from_host(w0)
    p1 = llk.PackedWeights.from_host(w1)
    dt = {"bf16": gpu.bfloat16, "f16": gpu.float16, "f32": gpu.float32}[c["out"]]
    with _Knobs(llk, tile_splits=c["splits"], decode_splits=c["splits"],
                decode_group_width=c["group"]):
        if c["op"] == "swiglu":
            yf = from_dev(llk.fused_swiglu(xd, p0, p1, out_dtype=gpu.float32))
            yo = from_dev(llk.fused_swiglu(xd, p0, p1, out_dtype=dt))
            ref, _ = orc.swiglu(x, w0, w1)
        else:
            yf = from_dev(llk.matmul(xd, p0, out_dtype=gpu.float32))
            yo = from_dev(llk.matmul(xd, p0, out_dtype=dt))
            ref, _ = orc.gemm(x, w0)
    assert_parity(yf, ref, f"random {i} fp32")
    if c["out"] == "bf16":
        assert np.array_equal(yo, to_bf16_bits(yf))
    elif c["out"] == "f16":
        assert np.array_equal(yo.view(np.uint16), yf.astype(np.float16).view(np.uint16))
    else:
        assert np.array_equal(yo, yf)
