"""sgpu_sgemm_splitk_noalloc -- sgpu_sgemm_splitk with its partial tiles and tile counters in
the library's fixed device scratch, allocating nothing -- through the C ABI, against
sgpu_sgemm_splitk (the same kernel with a per-stream workspace) and the oracle.

Bars: bit-identical to sgpu_sgemm_splitk at the same split count; reference-generator inputs
within max|C - C_ref| / max|C_ref| <= 1e-4 of the oracle (og_sgemm, gpu_workload.c:97-98);
integer inputs exact.  Two calls in a row, the second smaller (the scratch keeps the first
call's partials and must not leak them into the second); problems past the scratch rejected."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run(gpu, fn, dA, dB, dC, M, N, K, S):
    dC.fill_bytes(0xFF)
    gpu.check(getattr(gpu.lib(), fn)(dA.ptr, dB.ptr, dC.ptr, M, N, K, S, None), fn)
    gpu.synchronize()
    return dC.to_host()


def test_noalloc_matches_splitk_reference_inputs(gpu, og):
    """srand(42) inputs (gpu_workload.c:81-82): the ragged 1023x1025x997 at 4 splits, then a
    smaller 300x200x500 at 3."""
    for M, N, K, S in [(1023, 1025, 997, 4), (300, 200, 500, 3)]:
        say(f"noalloc splitk srand {M}x{N}x{K} S={S}")
        A, B = gpu.gen_sgemm_inputs(max(M * K, K * N), 42)
        A, B = A[:M * K], B[:K * N]
        dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
        want = run(gpu, "sgpu_sgemm_splitk", dA, dB, dC, M, N, K, S)
        got = run(gpu, "sgpu_sgemm_splitk_noalloc", dA, dB, dC, M, N, K, S)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        ref = og.sgemm_rows(A, B, M, N, K, 0, M, NT).astype(np.float64)
        assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-4


def test_noalloc_integer_exact_two_calls(gpu):
    """Integer inputs: the largest K-tailed problem the scratch holds at 4 splits
    (1408x1408x997: 484 tiles, 1936 of 2048 tile-splits), then a small one with more splits
    than slices (reduced to one slice per split)."""
    rng = np.random.default_rng(29)
    for M, N, K, S in [(1408, 1408, 997, 4), (33, 17, 96, 64)]:
        say(f"noalloc splitk integer {M}x{N}x{K} S={S}")
        A = rng.integers(-2, 3, (M, K)).astype(np.float32)
        B = rng.integers(-2, 3, (K, N)).astype(np.float32)
        dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
        got = run(gpu, "sgpu_sgemm_splitk_noalloc", dA, dB, dC, M, N, K, S)
        assert np.array_equal(got, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))
        assert np.array_equal(got, run(gpu, "sgpu_sgemm_splitk", dA, dB, dC, M, N, K, S))


def test_noalloc_rejects_problems_past_the_scratch(gpu):
    """4096^3 at 2 splits needs 4096 tiles x 2 x 4096 floats (128 MiB) of partials: rejected
    before any launch, with an error naming the scratch; C untouched."""
    M = N = K = 4096
    dC = gpu.DeviceArray(4)
    dC.fill_bytes(0x7F)
    rc = gpu.lib().sgpu_sgemm_splitk_noalloc(dC.ptr, dC.ptr, dC.ptr, M, N, K, 2, None)
    assert rc == gpu.SGPU_ERR_SCRATCH_LIMIT
    assert "scratch" in gpu.error_string(rc)
    rc = gpu.lib().sgpu_sgemm_splitk_noalloc(dC.ptr, dC.ptr, dC.ptr, 64, 64 * 16385, 64, 1, None)
    assert rc == gpu.SGPU_ERR_SCRATCH_LIMIT                  # more tiles than counters
    assert gpu.lib().sgpu_sgemm_splitk_noalloc(None, None, None, 0, 5, 5, 1, None) == 0      # empty: no-op
    gpu.synchronize()
    assert np.array_equal(dC.to_host().view(np.uint32), np.full(4, 0x7F7F7F7F, np.uint32))
