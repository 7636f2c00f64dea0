"""sgpu_sgemm_opt's launch plan (sgpu_sgemm_opt_plan), host logic only: no device is touched.

The pinned table holds the picks at MI355X's 256 CUs.  The split counts there come from the
library's cost model, whose measured basis is in the comment above splitk_pick in
csrc/sgpu.c, so a change to the model or a rule shows up here.  The invariants are what every
plan must satisfy at any CU count.  One of them, the split-K workspace bound, is what
sgpu_sgemm_splitk itself enforces."""
import ctypes as ct
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "switch-l4t-gpu_amd"))

import sgpu  # noqa: E402

PINNED_256 = [
    # whole rounds of 128x128 tiles (the last at least 94% full) with K >= 512 (K >= 4096 where
    # the busiest-CU model picks sgemm_opt256): the 128x128 K-over-waves member
    (4096, 4096, 4096, "sgemm_kwave128", 1),
    (8192, 8192, 8192, "sgemm_kwave128", 1),
    (2048, 2048, 2048, "sgemm_kwave128", 1),
    (2048, 2048, 512, "sgemm_kwave128", 1),
    (6144, 6144, 1024, "sgemm_kwave128", 1),
    (2048, 4096, 2048, "sgemm_kwave128", 1),
    (2816, 2816, 2816, "sgemm_kwave128", 1),
    (4096, 4096, 8192, "sgemm_kwave128", 1),
    # large problems: the member whose busiest CU has the least work; where that is the 64x64
    # member (several rounds of 64x64 tiles, K >= 256) the K-over-waves members run its tiles
    (4096, 4096, 1024, "sgemm_opt256", 1),
    (4096, 4096, 2048, "sgemm_opt256", 1),
    (2048, 8192, 1024, "sgemm_opt256", 1),
    (2048, 2048, 256, "sgemm_tiled4", 1),
    (5120, 5120, 5120, "sgemm_kwave", 1),
    (4096, 4096, 4064, "sgemm_opt256", 1),
    (4096, 4096, 4080, "sgemm_opt256", 1),
    (3072, 3072, 3072, "sgemm_kwave", 1),
    (2048, 1024, 1024, "sgemm_kwave", 1),
    (4097, 4097, 4097, "sgemm_kwave_edge", 1),
    (2047, 2049, 2047, "sgemm_kwave_edge", 1),
    (1408, 1408, 997, "sgemm_kwave_edge", 1),
    (2048, 1024, 1000, "sgemm_kwave_edge", 1),
    # one round of 64x64 tiles filling 3/4 of the CUs or more, K >= 256: the K-over-waves
    # members (whole tiles, or clamped edge tiles and a partial first k-slice)
    (1024, 1024, 1024, "sgemm_kwave", 1),
    (1024, 1024, 4096, "sgemm_kwave", 1),
    (1024, 768, 1024, "sgemm_kwave", 1),
    (1024, 1024, 992, "sgemm_kwave", 1),
    (1024, 1024, 512, "sgemm_kwave", 1),
    (1024, 1024, 256, "sgemm_kwave", 1),
    (1023, 1025, 997, "sgemm_kwave_edge", 1),
    (1000, 1000, 1000, "sgemm_kwave_edge", 1),
    (1024, 1024, 1000, "sgemm_kwave_edge", 1),
    (8192, 128, 1000, "sgemm_kwave_edge", 1),
    (1000, 1000, 384, "sgemm_kwave_edge", 1),
    (1000, 1000, 256, "sgemm_kwave_edge", 1),
    # K under 256: the 64x64 member, or the edge member from K 128 when N % 64 == 1 would give
    # the 64x64 member a second round
    (1024, 1024, 128, "sgemm_tiled", 1),
    (1000, 1000, 192, "sgemm_tiled", 1),
    (1023, 1025, 128, "sgemm_kwave_edge", 1),
    (1023, 1025, 64, "sgemm_tiled", 1),
    # fewer tiles: K splits across blocks
    (768, 768, 2048, "sgemm_splitk", 5),
    (512, 1024, 1024, "sgemm_splitk", 2),
    (1088, 1024, 1024, "sgemm_splitk", 4),
    (640, 640, 1000, "sgemm_splitk", 5),
    (1087, 1085, 2000, "sgemm_splitk", 7),
    # few tiles: tall K splits up to 16 ways, one row or column of tiles
    (64, 64, 8192, "sgemm_splitk", 16),
    (32, 32, 16384, "sgemm_splitk", 16),
    (256, 256, 4096, "sgemm_splitk", 8),
    (8192, 1, 2048, "sgemm_splitk", 2),
    (1, 8192, 4096, "sgemm_splitk", 4),
    # the small members
    (256, 256, 256, "sgemm_small16", 1),
    (512, 512, 512, "sgemm_small32", 1),
    (1, 4096, 4096, "sgemm_small16", 1),
    (16, 4096, 4096, "sgemm_small16", 1),
    (100, 70, 3000, "sgemm_small16", 1),
]


def plan(M, N, K, cus):
    s = ct.c_int(-1)
    name = sgpu.lib().sgpu_sgemm_opt_plan(M, N, K, cus, ct.byref(s))
    return (name.decode() if name else None), s.value


@pytest.mark.parametrize("M,N,K,name,S", PINNED_256)
def test_plan_pinned_at_256_cus(M, N, K, name, S):
    assert plan(M, N, K, 256) == (name, S)


def cdiv(a, b):
    return -(-a // b)


@pytest.mark.parametrize("cus", [1, 80, 104, 256, 304])
def test_plan_invariants(cus):
    members = {"sgemm_opt256", "sgemm_opt", "sgemm_tiled4", "sgemm_tiled", "sgemm_kwave", "sgemm_kwave_edge",
               "sgemm_kwave128"}
    for M in (1, 17, 64, 300, 1000, 1023, 2048):
        for N in (1, 64, 511, 1000, 1025, 4096):
            for K in (0, 1, 31, 64, 128, 320, 997, 2048, 8192):
                name, S = plan(M, N, K, cus)
                tiles = cdiv(M, 64) * cdiv(N, 64)
                nk = cdiv(K, 32)
                if name == "sgemm_splitk":
                    assert 2 <= S <= 16 and K > 0
                    per = cdiv(nk, S)
                    assert cdiv(nk, per) == S            # S is already the reduced split count
                    assert per >= 2                       # every split holds two slices or more
                    assert S * tiles * 4096 <= 8 << 20    # the 32 MB workspace
                    assert tiles <= 2 * cus
                    assert S <= 8 or (tiles * 2 <= cus and K // 16 >= 512)
                else:
                    assert S == 1
                    if name == "sgemm_small16":
                        assert cdiv(M, 16) * cdiv(N, 16) <= cus and K <= 4096
                    elif name == "sgemm_small32":
                        assert cdiv(M, 32) * cdiv(N, 32) <= cus and K <= 1024
                    elif name == "sgemm_kwave":
                        assert M % 64 == 0 and N % 64 == 0 and K % 32 == 0 and K >= 256
                    elif name == "sgemm_kwave128":
                        t128 = (M // 128) * (N // 128)
                        assert M % 128 == 0 and N % 128 == 0 and K % 32 == 0 and K >= 512
                        assert 50 * t128 >= 47 * cdiv(t128, cus) * cus
                    elif name == "sgemm_kwave_edge":
                        assert M >= 64 and N >= 64 and K >= 128
                        assert M % 64 or N % 64 or K % 32
                        edge_tiles = cdiv(M, 64) * (N // 64 if N % 64 == 1 else cdiv(N, 64))
                        if K < 256:
                            assert edge_tiles <= cus and 4 * edge_tiles >= 3 * cus and tiles > cus
                    else:
                        assert name in members
                        if name == "sgemm_tiled" and M >= 64 and N >= 64:
                            assert K < 256                        # else the K-over-waves members run its tiles


def test_plan_rejects():
    assert plan(0, 4, 4, 256) == (None, -1)
    assert plan(4, 0, 4, 256) == (None, -1)
    assert plan(4, 4, -1, 256) == (None, -1)
    assert plan(4, 4, 4, 0) == (None, -1)
    assert sgpu.lib().sgpu_sgemm_opt_plan(64, 64, 64, 256, None) is not None


def test_bench_traffic_record_covers_the_4096_member():
    """bench.py reports the HBM traffic of the member sgpu_sgemm_opt launches at 4096^3 from
    profiles/traffic.json under "<member>_4096"; a plan change that moves 4096^3 to another
    member needs that member's PMC record, or the bench line's roofline.traffic goes null."""
    import json

    name, _ = plan(4096, 4096, 4096, 256)
    rec = json.load(open(os.path.join(ROOT, "profiles", "traffic.json")))
    assert f"{name}_4096" in rec
    assert rec[f"{name}_4096"] >= 3 * 4 * 4096 * 4096          # at least A, B and C once
    assert "gemv_h_lm_head" in rec and "gemv_hh_lm_head" in rec
