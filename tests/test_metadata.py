"""CPU tests: integer metadata of the path must match the reference exactly
(M buckets, tiling helpers, KernelKey hash, packWeightMatrix metadata and
host layout, schedule-DB lookup)."""
from __future__ import annotations

import ctypes as C
import json
from pathlib import Path

import numpy as np
import pytest

from common import normal_bf16

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------------------
# classifyM
# ---------------------------------------------------------------------------

# specialization_dispatch.cpp:32-62 (M, expected bucket) and
# shape_specialization.mlir:10-46 (M=1,4,16,64,128 -> 0..4).
BUCKETS = [(1, 0), (2, 1), (4, 1), (5, 2), (8, 2), (16, 2), (17, 3), (32, 3), (64, 3), (65, 4),
           (128, 4), (512, 4), (3, 1), (4096, 4)]


@pytest.mark.parametrize("M,bucket", BUCKETS)
def test_classify_m(llk, orc, M, bucket):
    assert llk.classify_m(M) == bucket
    assert orc.orc().orc_classify_m(M) == bucket


def test_classify_m_nonpositive(llk):
    """ScheduleLoader.cpp:19-29 sends M <= 0 to bucket 1 (the test-local copy
    in specialization_dispatch.cpp:15-25 would say 4); the library follows
    the loader the compiler uses."""
    assert llk.classify_m(0) == 1 and llk.classify_m(-5) == 1


def test_baseline_config_buckets(llk):
    """Buckets of the BASELINE configurations."""
    assert [llk.classify_m(m) for m in (64, 2048, 1, 8, 16, 17, 255, 1000, 4097)] == \
        [3, 4, 0, 2, 2, 3, 4, 4, 4]


# ---------------------------------------------------------------------------
# TilingUtils.h:28-50
# ---------------------------------------------------------------------------

def test_tiling_helpers(llk, orc):
    L, O = llk.lib(), orc.orc()
    cases = [(2048, 32), (11008, 64), (127, 8), (0, 32), (5, 0), (64, 64), (65, 64)]
    expect_num = [64, 172, 16, 0, 1, 1, 2]
    for (d, t), e in zip(cases, expect_num):
        assert L.llk_num_tiles(d, t) == e == O.orc_num_tiles(d, t)
    # last tile short, past-the-end tiles empty
    assert L.llk_tile_size(127, 8, 15) == 7 and L.llk_tile_size(127, 8, 16) == 0
    assert L.llk_tile_size(64, 32, 1) == 32
    assert L.llk_num_inner_tiles(64, 8) == 8 and L.llk_num_inner_tiles(63, 8) == 8
    assert L.llk_num_inner_tiles(10, 0) == 1
    for d in range(0, 70):
        for t in (1, 7, 32):
            n = L.llk_num_tiles(d, t)
            assert sum(L.llk_tile_size(d, t, i) for i in range(n + 1)) == d


# ---------------------------------------------------------------------------
# KernelKey::hash (KernelKey.h:60-86)
# ---------------------------------------------------------------------------

def _random_keys(n, seed=0):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        yield (int(rng.integers(0, 3)), int(rng.integers(0, 3)), int(rng.integers(0, 3)),
               int(rng.integers(-1, 5)), int(rng.integers(0, 1 << 20)), int(rng.integers(0, 1 << 20)),
               int(rng.integers(0, 2)), int(rng.integers(0, 7)), int(rng.integers(0, 3)),
               int(rng.integers(0, 1 << 16)), int(rng.integers(0, 1 << 62)),
               int(rng.integers(0, 1 << 62)))


def test_kernel_key_hash_matches_reference_header(llk, orc):
    """Against llk::KernelKey::hash compiled from the reference's own header
    (oracle/_ref), on 500 random keys and the default key."""
    ref = orc.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    L = llk.lib()
    for k in _random_keys(500):
        h = L.llk_kernel_key_hash(*k)
        assert h == ref.ref_kernel_key_hash(*k) == orc.orc().orc_kernel_key_hash(*k)
    # default-initialised key: op 0, bf16, bf16, 0, 0, 0, row-major, AVX2,
    # bounded_fast (1), threads 1, versions 0 (KernelKey.h:45-57)
    assert L.llk_kernel_key_hash(0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 0, 0) == \
        ref.ref_kernel_key_default_hash()


def test_kernel_key_hash_properties(llk):
    """schedule_determinism.cpp:15-83 and jit_cache_hit.cpp:20-71: equal keys
    hash equal, and changing op / bucket / N / K / threads / schedule version
    changes the hash."""
    L = llk.lib()
    base = [0, 0, 0, 2, 4096, 4096, 0, 0, 1, 8, 0, 0]
    h0 = L.llk_kernel_key_hash(*base)
    assert all(L.llk_kernel_key_hash(*base) == h0 for _ in range(100))
    for idx, val in [(0, 1), (3, 3), (4, 11008), (5, 2048), (9, 4), (11, 2), (7, 7)]:
        k = list(base)
        k[idx] = val
        assert L.llk_kernel_key_hash(*k) != h0
    ops = {L.llk_kernel_key_hash(op, 0, 0, 0, 0, 0, 0, 0, 1, 1, 0, 0) for op in range(4)}
    assert len(ops) == 4


# ---------------------------------------------------------------------------
# PackedWeights (PackedWeights.cpp:5-37)
# ---------------------------------------------------------------------------

# (K, N, BK) -> (K_blocks, block_size) for the BASELINE matrices.
PACK_META = [((512, 1376, 64), (8, 176128)), ((4096, 11008, 64), (64, 1409024)),
             ((4096, 14336, 64), (64, 1835008)), ((5120, 13824, 64), (80, 1769472)),
             ((13824, 5120, 64), (216, 655360)), ((100, 30, 64), (2, 3840)),
             ((3, 8, 64), (1, 1024)), ((130, 7, 32), (5, 448))]


@pytest.mark.parametrize("dims,meta", PACK_META)
def test_pack_metadata(llk, orc, dims, meta):
    K, N, BK = dims
    m = np.zeros(5, np.int64)
    orc.orc().orc_pack_weight_meta(K, N, BK, m)
    assert (int(m[0]), int(m[2])) == meta
    if K * N <= 200_000:
        w = normal_bf16(1, 1, (K, N))
        pw = llk.PackedWeights.from_host(w, bk=BK, host_only=True)
        assert (pw.K_blocks, pw.N, pw.block_size, pw.BK, pw.dtype) == (meta[0], N, meta[1], BK, 0)
        pw.free()


def test_pack_host_layout_matches_oracle_and_row_major(llk, orc):
    """The reference host layout [K_blocks][BK][N] (zero-padded) equals the
    oracle's restatement, and equals the row-major matrix when K % BK == 0
    (PackedWeights.cpp:23-31)."""
    for (K, N, BK) in [(128, 40, 64), (130, 40, 64), (7, 5, 4)]:
        w = normal_bf16(2, 1, (K, N))
        pw = llk.PackedWeights.from_host(w, bk=BK, host_only=True)
        host = pw.host_data()
        ref_layout, _ = orc.pack_weight_matrix(w, BK)
        assert np.array_equal(host, ref_layout)
        flat = host.reshape(-1, N)
        assert np.array_equal(flat[:K], w) and not flat[K:].any()
        # repack keeps BK and replaces the contents
        w2 = normal_bf16(3, 1, (K, N))
        pw.repack(w2)
        assert pw.BK == BK and np.array_equal(pw.host_data().reshape(-1, N)[:K], w2)
        pw.free()


def test_pack_strided_source(llk):
    """stride0 > N: rows are taken from w + k*stride0 (PackedWeights.cpp:20)."""
    big = normal_bf16(4, 1, (70, 50))
    view = big[:, 3:43]
    pw = llk.PackedWeights.from_host(view, bk=16, host_only=True)
    assert np.array_equal(pw.host_data().reshape(-1, 40)[:70], view)


def test_device_layout_mapping(llk):
    """The device payload (1 KiB v_mfma_f32_32x32x16_bf16 A operands) follows
    the documented mapping: element W[k][n] of block (nb, kb) sits in
    sub-block (k%64)//16*4 + (n%128)//32, lane ((k%16)//8)*32 + n%32, slot k%8."""
    K, N = 130, 200
    w = normal_bf16(5, 1, (K, N))
    dev = llk.pack_device_layout(w).view(np.uint16)
    KB, NB = -(-K // 64), -(-N // 128)
    assert dev.size == KB * NB * 8192
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    pos = (((n // 128) * KB + k // 64) * 8192 + ((k % 64) // 16 * 4 + (n % 128) // 32) * 512 +
           (((k % 16) // 8) * 32 + n % 32) * 8 + k % 8)
    assert np.array_equal(dev[pos], w)
    mask = np.ones(dev.size, bool)
    mask[pos.ravel()] = False
    assert not dev[mask].any()  # padding is zero


# ---------------------------------------------------------------------------
# Schedule DB (ScheduleLoader.cpp:31-98, ScheduleSelection.cpp:46-67)
# ---------------------------------------------------------------------------

DB = str(GOLDEN / "schedule_db_reference.json")  # copy of the reference's schedules/schedule_db.json

# (op, bucket) -> (BM, BN, BK, VM, VN, vector_width, threads, grain, axis, n_matches):
# first matching entry of schedule_db.json (lines cited), N and K ignored.
SCHED = {
    ("fused_swiglu", 0): ((1, 64, 64, 1, 8, 8, 8, 1, "n"), 2),     # :4-18 (and :202-219)
    ("fused_swiglu", 1): ((4, 64, 64, 1, 8, 8, 4, 1, "n"), 1),     # :19-33
    ("fused_swiglu", 2): ((8, 64, 64, 2, 8, 8, 8, 2, "m"), 5),     # :34-48 (+4 later entries)
    ("fused_swiglu", 3): ((16, 64, 64, 4, 8, 8, 8, 2, "m"), 1),    # :49-63
    ("fused_swiglu", 4): ((32, 64, 64, 4, 8, 8, 8, 4, "m"), 2),    # :64-78 (and :220-236)
}


@pytest.mark.parametrize("key", sorted(SCHED))
def test_schedule_lookup_reference_db(llk, key):
    op, bucket = key
    e, n, st = llk.select_schedule(DB, op, bucket)
    want, nmatch = SCHED[key]
    got = (e.BM, e.BN, e.BK, e.VM, e.VN, e.vector_width, e.num_threads, e.grain_size,
           e.parallel_axis.decode())
    assert st == 0 and got == want and n == nmatch


def test_schedule_lookup_matches_db_contents(llk):
    """Every (operation, bucket) pair: the library returns the first entry of
    the file with that operation and bucket, whatever N/K/target say."""
    db = json.load(open(DB))
    for op in ("fused_swiglu", "rope", "attention", "nope"):
        for bucket in range(-1, 6):
            matches = [e for e in db["entries"] if e.get("operation") == op and
                       e["shape"].get("M_bucket") == bucket and "N" in e["shape"] and
                       "K" in e["shape"]]
            e, n, st = llk.select_schedule(DB, op, bucket)
            assert n == len(matches)
            if matches:
                s = matches[0]["schedule"]
                assert (e.BM, e.BN, e.BK, e.num_threads) == (s["BM"], s["BN"], s["BK"],
                                                             s.get("num_threads", 1))
            else:
                assert (e.BM, e.BN, e.BK, e.VM, e.VN, e.num_threads) == (8, 32, 32, 1, 4, 4)


def test_schedule_lookup_fallbacks(llk, tmp_path):
    """Missing or invalid file: warn-and-fall-back (ScheduleLoader.cpp:36-46)
    -> default schedule and LLK_ERR_NOT_FOUND.  Entries without N/K, or with
    a non-integer bucket, are skipped; missing integers default to 0 / 1."""
    e, n, st = llk.select_schedule(str(tmp_path / "missing.json"), "fused_swiglu", 0)
    assert st == -11 and n == 0 and (e.BM, e.BN, e.BK, e.parallel_axis) == (8, 32, 32, b"n")
    bad = tmp_path / "bad.json"
    bad.write_text("{ not json")
    e, n, st = llk.select_schedule(str(bad), "fused_swiglu", 0)
    assert st == -11 and e.BM == 8
    p = tmp_path / "db.json"
    p.write_text(json.dumps({"entries": [
        {"operation": "fused_swiglu", "shape": {"M_bucket": 0, "N": 1}, "schedule": {"BM": 99}},
        {"operation": "fused_swiglu", "shape": {"M_bucket": 0.5, "N": 1, "K": 1},
         "schedule": {"BM": 98}},
        {"operation": "fused_swiglu", "shape": {"M_bucket": 0, "N": 1, "K": 2},
         "schedule": {"BM": 7, "parallel_axis": "m"}},
    ]}))
    e, n, st = llk.select_schedule(str(p), "fused_swiglu", 0)
    assert st == 0 and n == 1
    assert (e.BM, e.BN, e.vector_width, e.num_threads, e.grain_size, e.parallel_axis) == \
        (7, 0, 0, 1, 1, b"m")


def test_gfx950_schedule_db(llk):
    """The backend's own schedules/gfx950 database uses the same record schema
    and covers every M bucket for fused_swiglu and matmul."""
    root = Path(llk.__file__).resolve().parent
    db = root / "schedules" / "gfx950" / "schedule_db.json"
    assert db.exists()
    for op in ("fused_swiglu", "matmul"):
        for bucket in range(5):
            e, n, st = llk.select_schedule(str(db), op, bucket)
            assert st == 0 and n >= 1, (op, bucket)
