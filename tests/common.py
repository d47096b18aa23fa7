"""Shared helpers for the test suite: deterministic inputs and parity metrics.

Input generator (used by tests and bench.py): counter-based splitmix64
streams with Box-Muller normals, scaled in fp32, rounded to bf16 with
round-to-nearest-even.  stream ids: X=0, Wg=1, Wu=2, Wd=3, outlier mask=4.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

STREAM_X, STREAM_WG, STREAM_WU, STREAM_WD, STREAM_MASK = 0, 1, 2, 3, 4


def splitmix64(seed: int, stream: int, n: int, offset: int = 0) -> np.ndarray:
    """z_i = mix(s0 + (offset + i + 1) * GOLDEN), s0 = seed ^ (stream * GOLDEN)."""
    with np.errstate(over="ignore"):
        s0 = np.uint64(seed) ^ (np.uint64(stream) * GOLDEN)
        idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = s0 + idx * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def normal_f32(seed: int, stream: int, n: int, sigma: float = 1.0) -> np.ndarray:
    """n standard normals (Box-Muller over splitmix64), times sigma, in fp32."""
    pairs = (n + 1) // 2
    z = splitmix64(seed, stream, 2 * pairs)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0 ** -53
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return out[:n].astype(np.float32) * np.float32(sigma)


def to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even (NaN kept quiet)."""
    b = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32)
    nan = (b & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    r = np.where(nan, (b >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16_np(seed: int, stream: int, shape, sigma: float = 1.0) -> np.ndarray:
    """numpy statement of the generator (cross-checks the library's C one)."""
    n = int(np.prod(shape))
    return to_bf16_bits(normal_f32(seed, stream, n, sigma)).reshape(shape)


def normal_bf16(seed: int, stream: int, shape, sigma: float = 1.0) -> np.ndarray:
    """bf16 bits of sigma * N(0,1) from the library's multithreaded generator
    (same definition as normal_bf16_np; a host function, no GPU needed)."""
    import dslcompiler_amd
    return dslcompiler_amd.fill_normal_bf16(seed, stream, tuple(shape), sigma)


def outliers(x_bits: np.ndarray, seed: int, frac: float = 0.01, scale: float = 20.0) -> np.ndarray:
    """Scales a seeded `frac` of the entries by `scale` (then re-rounds)."""
    z = splitmix64(seed, STREAM_MASK, x_bits.size)
    u = (z >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    f = bf16_bits_to_f32(x_bits).ravel().copy()
    f[u < frac] *= np.float32(scale)
    return to_bf16_bits(f).reshape(x_bits.shape)


def swiglu_inputs(M: int, K: int, N: int, seed: int = 42):
    """X ~ N(0,1), Wg, Wu ~ N(0, 1/sqrt(K)) as bf16 bits."""
    x = normal_bf16(seed, STREAM_X, (M, K))
    s = 1.0 / np.sqrt(K)
    wg = normal_bf16(seed, STREAM_WG, (K, N), s)
    wu = normal_bf16(seed, STREAM_WU, (K, N), s)
    return x, wg, wu


def parity(got: np.ndarray, want: np.ndarray) -> dict:
    """rel-L2 and max-abs / RMS(want), in float64."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    diff = g - w
    rms = float(np.sqrt(np.mean(w * w))) if w.size else 0.0
    l2w = float(np.linalg.norm(w))
    rel_l2 = float(np.linalg.norm(diff)) / l2w if l2w > 0 else float(np.linalg.norm(diff))
    maxabs = float(np.max(np.abs(diff))) if diff.size else 0.0
    return {"rel_l2": rel_l2, "max_abs": maxabs, "rms": rms,
            "max_abs_over_rms": maxabs / rms if rms > 0 else maxabs}


# The bar of the north star: relative L2 <= 1e-3 and max-abs <= 2e-2 * RMS.
REL_L2_TOL = 1e-3
MAX_ABS_RMS_TOL = 2e-2


def assert_parity(got, want, what: str = "") -> dict:
    p = parity(got, want)
    assert p["rel_l2"] <= REL_L2_TOL, f"{what}: rel-L2 {p['rel_l2']:.3e} > {REL_L2_TOL}"
    assert p["max_abs_over_rms"] <= MAX_ABS_RMS_TOL, (
        f"{what}: max-abs/RMS {p['max_abs_over_rms']:.3e} > {MAX_ABS_RMS_TOL}")
    return p


# A bf16 result may differ from the oracle's RNE(fp32) by one ulp where the
# oracle's fp32 value lies within this relative distance of the midpoint
# between two bf16 neighbours: fp32 sums taken in a different order differ by
# ~1e-6 relative (more for long reductions: K = 13824 in config 5), so such
# elements round either way.  At most this fraction of elements may be
# boundary flips; each one is verified individually.
FLIP_MIDPOINT_REL = 1e-4
FLIP_MAX_FRACTION = 1e-2


def assert_parity_bf16(got_bits: np.ndarray, ref_f32: np.ndarray, what: str = "") -> dict:
    """bf16 output against the oracle: rel-L2 <= 1e-3 versus the oracle's
    bf16 (RNE of its fp32), and max-abs <= 2e-2 * RMS over all elements except
    rounding-boundary flips, which must each be the other bf16 neighbour of
    the oracle's fp32 value with that value within FLIP_MIDPOINT_REL of the
    rounding midpoint.  Returns the metrics, including the raw max-abs."""
    got = bf16_bits_to_f32(got_bits).astype(np.float64)
    ref_bits = to_bf16_bits(ref_f32)
    ref = bf16_bits_to_f32(ref_bits).astype(np.float64)
    rf = np.asarray(ref_f32, np.float64)
    p = parity(got, ref)
    assert p["rel_l2"] <= REL_L2_TOL, f"{what}: rel-L2 {p['rel_l2']:.3e} > {REL_L2_TOL}"
    diff = got_bits.astype(np.int32) != ref_bits.astype(np.int32)
    flips = np.zeros_like(diff)
    if diff.any():
        g, r, f = got[diff], ref[diff], rf[diff]
        mid = 0.5 * (g + r)
        # adjacent bf16 numbers (same sign) that bracket the fp32 value
        bracket = (np.minimum(g, r) <= f) & (f <= np.maximum(g, r))
        adjacent = np.abs(got_bits[diff].astype(np.int32) - ref_bits[diff].astype(np.int32)) == 1
        near_mid = np.abs(f - mid) <= FLIP_MIDPOINT_REL * np.maximum(np.abs(f), 1e-30)
        ok = bracket & adjacent & near_mid
        flips[diff] = ok
    n_flip = int(flips.sum())
    p["boundary_flips"] = n_flip
    p["raw_max_abs_over_rms"] = p["max_abs_over_rms"]
    assert n_flip <= max(1, FLIP_MAX_FRACTION * got.size), (
        f"{what}: {n_flip} boundary flips in {got.size} elements")
    kept = ~flips
    maxabs = float(np.max(np.abs(got - ref)[kept])) if kept.any() else 0.0
    p["max_abs_over_rms"] = maxabs / p["rms"] if p["rms"] > 0 else maxabs
    assert p["max_abs_over_rms"] <= MAX_ABS_RMS_TOL, (
        f"{what}: max-abs/RMS {p['max_abs_over_rms']:.3e} > {MAX_ABS_RMS_TOL} "
        f"(excluding {n_flip} boundary flips)")
    return p
