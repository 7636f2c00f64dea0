"""SGEMM family on the GPU through the C ABI, against the oracle (og_sgemm, restating
gpu_workload.c:97-98) and exact integer arithmetic.

Bars: reference-generator inputs (srand(42), gpu_workload.c:81-82) at every size
max|C - C_ref| / max|C_ref| <= 1e-4 and the reference verdict (5% + 1e-3) clean; small-integer
inputs (|a|, |b| <= 2, every partial sum an exact fp32 integer) bit-exact against float64
BLAS at every shape, including ragged edges and the full 4096^3."""
import ctypes as ct
import functools
import json
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin")
VARIANTS = ["sgpu_sgemm_tiled", "sgpu_sgemm_tiled4", "sgpu_sgemm_opt", "sgpu_sgemm_naive"]
NORMWISE_TOL = 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run_sgemm(gpu, fn, A, B, M, N, K, a_off=0, b_off=0):
    """C = A B through launcher `fn`; a_off/b_off shift the operands by whole floats to
    exercise unaligned base pointers.  C is pre-filled with NaN so unwritten cells show."""
    dA = gpu.DeviceArray(M * K + a_off + 1)
    dB = gpu.DeviceArray(K * N + b_off + 1)
    if A.size:
        gpu.call("sgpu_memcpy_htod", dA.offset(a_off), np.ascontiguousarray(A, np.float32).ctypes.data, A.size * 4)
    if B.size:
        gpu.call("sgpu_memcpy_htod", dB.offset(b_off), np.ascontiguousarray(B, np.float32).ctypes.data, B.size * 4)
    dC = gpu.DeviceArray((M, N))
    dC.fill_bytes(0xFF)
    gpu.call(fn, dA.offset(a_off), dB.offset(b_off), dC.ptr, M, N, K, None)
    gpu.synchronize()
    return dC.to_host()


@functools.lru_cache(maxsize=None)
def ref_inputs(M, N, K):
    from sgpu import gen_sgemm_inputs

    n = max(M * K, K * N)
    A, B = gen_sgemm_inputs(n, 42)
    return A[:M * K].reshape(M, K), B[:K * N].reshape(K, N)


@functools.lru_cache(maxsize=None)
def ref_golden(M, N, K):
    import oracle

    A, B = ref_inputs(M, N, K)
    return oracle.sgemm_rows(A, B, M, N, K, 0, M, nthreads=min(16, os.cpu_count() or 1))


@pytest.mark.parametrize("n", [256, 512, 1024])
@pytest.mark.parametrize("fn", VARIANTS)
def test_reference_generator(gpu, og, fn, n):
    say(f"sgemm {fn} n={n} reference inputs")
    A, B = ref_inputs(n, n, n)
    C = run_sgemm(gpu, fn, A, B, n, n, n)
    ref = ref_golden(n, n, n)
    err = np.abs(C.astype(np.float64) - ref).max() / np.abs(ref).max()
    assert err <= NORMWISE_TOL, err
    assert og.sgemm_verdict_bad(C, ref, n, n) == 0


@pytest.mark.parametrize("fn", VARIANTS[:3])
def test_ragged_reference_generator(gpu, og, fn):
    M, N, K = 1023, 1025, 997
    say(f"sgemm {fn} ragged {M}x{N}x{K}")
    A, B = ref_inputs(M, N, K)
    C = run_sgemm(gpu, fn, A, B, M, N, K)
    ref = ref_golden(M, N, K)
    assert np.abs(C.astype(np.float64) - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    assert og.sgemm_verdict_bad(C, ref, M, N) == 0


SHAPES = [(1, 1, 1), (3, 5, 7), (64, 64, 16), (65, 33, 17), (127, 129, 131), (128, 128, 1), (256, 256, 256),
          (300, 200, 64), (1023, 1025, 997), (257, 511, 1030)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("fn", VARIANTS)
def test_integer_exact(gpu, fn, M, N, K):
    say(f"sgemm {fn} integer {M}x{N}x{K}")
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    C = run_sgemm(gpu, fn, A, B, M, N, K)
    assert np.array_equal(C, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))


# Shapes that steer sgpu_sgemm_opt to each member and each member to both its pipelined path
# (M, N whole tiles, K whole slices, at least two slices) and its bounds-checked path.
DISPATCH_SHAPES = [(2048, 8192, 48), (2048, 8192, 32), (2047, 8191, 50), (4096, 4096, 16),
                   (2048, 4096, 64), (2048, 4096, 96), (256, 256, 64), (192, 320, 40),
                   (4096, 4096, 96), (4096, 4352, 64), (4352, 4096, 160),
                   # sgpu_sgemm_opt's small-member and split-K regimes: one row or column of
                   # tiles (the 16x16 member at 4096 wide, split-K at 8192), two rounds of
                   # K-tailed 64x64 tiles left unsplit, and a 7-way split of 289 tiles (2023
                   # partial tiles, 31.6 MB: near the workspace's 2048)
                   (1, 4096, 4096), (4096, 1, 2048), (1, 8192, 4096), (8192, 1, 2048), (1408, 1408, 997),
                   (1087, 1085, 2000),
                   # the small members' K bounds and the 16-way split of one tall-K tile
                   (256, 256, 4096), (100, 70, 3000), (16, 4096, 4096), (64, 64, 8192),
                   # one round of 64x64 tiles split 5 ways, one on the K-over-waves member and
                   # three on its edge form (one column past the whole tiles; clamped edges)
                   (768, 768, 2048), (1024, 768, 1024), (1023, 1025, 997), (1000, 1000, 1000), (8192, 128, 1000)]


@pytest.mark.parametrize("M,N,K", DISPATCH_SHAPES)
@pytest.mark.parametrize("fn", ["sgpu_sgemm_opt", "sgpu_sgemm_opt256", "sgpu_sgemm_tiled4", "sgpu_sgemm_tiled"])
def test_tile_paths_integer_exact(gpu, fn, M, N, K):
    say(f"sgemm {fn} integer {M}x{N}x{K}")
    rng = np.random.default_rng(M + N * 3 + K * 11)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    C = run_sgemm(gpu, fn, A, B, M, N, K)
    assert np.array_equal(C, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))


# sgpu_sgemm_opt launches what sgpu_sgemm_opt_plan names for this device: on float inputs its
# C equals the named launch's bit for bit.  A split sums its partials in split order, so a
# split C differs from the unsplit member's, and a different split count would differ too.
PLAN_SHAPES = [(1023, 1025, 997), (768, 768, 2048), (1000, 1000, 1000), (1088, 1024, 1024), (1024, 1024, 1000),
               (8192, 128, 1000), (1023, 1025, 128),
               (2048, 1024, 1000), (640, 640, 4096), (64, 64, 8192), (256, 256, 256), (512, 512, 512),
               (1024, 1024, 1024), (2048, 2048, 2048)]


@pytest.mark.parametrize("M,N,K", PLAN_SHAPES)
def test_opt_launches_its_plan(gpu, M, N, K):
    import ctypes as ct

    cus = gpu.device_props().compute_units
    S = ct.c_int()
    name = gpu.lib().sgpu_sgemm_opt_plan(M, N, K, cus, ct.byref(S)).decode()
    say(f"sgemm_opt plan {M}x{N}x{K} on {cus} CUs: {name} S={S.value}")
    A, B = ref_inputs(M, N, K)
    dA, dB = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B)
    dC, dD = gpu.DeviceArray((M, N)), gpu.DeviceArray((M, N))
    dC.fill_bytes(0xFF)
    dD.fill_bytes(0xFF)
    gpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
    if name == "sgemm_splitk":
        gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dD.ptr, M, N, K, S.value, None)
    elif name in ("sgemm_small16", "sgemm_small32"):
        gpu.call("sgpu_sgemm_small", dA.ptr, dB.ptr, dD.ptr, M, N, K, int(name[-2:]), None)
    else:
        gpu.call("sgpu_" + name, dA.ptr, dB.ptr, dD.ptr, M, N, K, None)
    gpu.synchronize()
    C = dC.to_host()
    assert np.array_equal(C, dD.to_host())
    if name == "sgemm_splitk":
        gpu.call("sgpu_sgemm_tiled", dA.ptr, dB.ptr, dD.ptr, M, N, K, None)
        gpu.synchronize()
        assert not np.array_equal(C, dD.to_host())


# Shapes whose edge tiles take the clamped-address path: an A tile (BM rows of K floats) or a
# B slice (BK rows of N floats) of 2^31 bytes or more.  Entries in {-1, 0, 1}: every partial
# sum is an exact fp32 integer (|sum| <= K < 2^24).
# The K-over-waves members: buffer offsets up to just under 2^31 bytes (a 64-row A panel of
# 64 * (2^23 - 32) floats, a 128-row one of 128 * (2^22 - 32)), the LDS-staged forms with 64-bit
# addresses past that (A of 2^31 bytes and more, with and without a K tail), and the extra
# column (N % 64 == 1) at 2^23 + 1 columns.
@pytest.mark.parametrize("fn,M,N,K", [("sgpu_sgemm_tiled", 3, 5, (1 << 23) + 7),
                                      ("sgpu_sgemm_opt256", 3, 5, (1 << 21) + 3),
                                      ("sgpu_sgemm_tiled", 2, (1 << 24) + 5, 3),
                                      ("sgpu_sgemm_kwave", 64, 64, (1 << 23) - 32),
                                      ("sgpu_sgemm_kwave", 64, 64, 1 << 23),
                                      ("sgpu_sgemm_kwave_edge", 64, 64, (1 << 23) + 7),
                                      ("sgpu_sgemm_kwave_edge", 64, (1 << 23) + 1, 65),
                                      ("sgpu_sgemm_kwave128", 128, 128, (1 << 22) - 32)])
def test_large_operand_windows_integer_exact(gpu, fn, M, N, K):
    say(f"sgemm {fn} large window {M}x{N}x{K}")
    rng = np.random.default_rng(K + N)
    A = rng.integers(-1, 2, (M, K)).astype(np.float32)
    B = rng.integers(-1, 2, (K, N)).astype(np.float32)
    C = run_sgemm(gpu, fn, A, B, M, N, K)
    assert np.array_equal(C, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))


# (M, N, K, S): even and uneven splits, K tails (a partial last slice), edge tiles, one tile
# with many splits, and S above the slice count (reduced to one slice per split).
SPLITK_CASES = [(512, 512, 512, 1), (512, 512, 512, 2), (512, 512, 512, 4), (512, 512, 512, 8),
                (1023, 1025, 997, 4), (100, 70, 3000, 8), (64, 64, 8192, 16), (257, 511, 1030, 3),
                (130, 260, 40, 5), (33, 17, 96, 64)]


@pytest.mark.parametrize("M,N,K,S", SPLITK_CASES)
def test_splitk_integer_exact(gpu, M, N, K, S):
    """Every split count gives the exact product on integer inputs, on two calls in a row
    (each launch leaves its tile counters at zero for the next)."""
    say(f"sgemm splitk integer {M}x{N}x{K} S={S}")
    rng = np.random.default_rng(M * 7 + N + K + S)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    for _ in range(2):
        dC.fill_bytes(0xFF)
        gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, S, None)
        gpu.synchronize()
        assert np.array_equal(dC.to_host(), want)


def test_splitk_streams_overlap(gpu):
    """Split-K launches on two streams, interleaved without synchronisation, and from two host
    threads on their own streams: each stream has its own workspace, so every result is the
    exact product (integer inputs) however the launches overlap on the device."""
    import threading

    M, N, K, S = 300, 260, 1100, 4
    rng = np.random.default_rng(17)
    mats = []
    for i in range(2):
        A = rng.integers(-2, 3, (M, K)).astype(np.float32)
        B = rng.integers(-2, 3, (K, N)).astype(np.float32)
        mats.append((gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N)),
                     (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)))
    streams = [gpu.Stream(), gpu.Stream()]
    say("split-K on two streams, interleaved")
    for _ in range(40):
        for (dA, dB, dC, _), st in zip(mats, streams):
            gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, S, st.h)
            gpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, M, N, K, st.h)
    gpu.synchronize()
    for dA, dB, dC, want in mats:
        assert np.array_equal(dC.to_host(), want)
    say("split-K from two host threads")
    errs = []

    def worker(i):
        dA, dB, dC, _ = mats[i]
        try:
            for _ in range(40):
                gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, S, streams[i].h)
            streams[i].synchronize()
        except Exception as e:          # reported below
            errs.append(e)

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs, errs
    for dA, dB, dC, want in mats:
        assert np.array_equal(dC.to_host(), want)
    for st in streams:
        st.close()


def test_splitk_recording_needs_a_workspace(gpu):
    """A stream being recorded cannot get a workspace: on a fresh stream sgpu_sgemm_splitk
    reports SGPU_ERR_NO_WORKSPACE and sgpu_sgemm_opt records its unsplit member; after one
    split launch outside recording, the stream's workspace is recorded and every replay is
    exact."""
    M, N, K = 768, 768, 2048                                # sgpu_sgemm_opt splits this one 5 ways
    rng = np.random.default_rng(19)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC, dD = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N)), \
        gpu.DeviceArray((M, N))
    st = gpu.Stream()
    with gpu.Graph(st) as g:
        rc = gpu.lib().sgpu_sgemm_splitk(dA.ptr, dB.ptr, dC.ptr, M, N, K, 4, st.h)
        gpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dD.ptr, M, N, K, st.h)
    assert rc == gpu.SGPU_ERR_NO_WORKSPACE
    assert "workspace" in gpu.error_string(rc)
    for _ in range(3):
        dD.fill_bytes(0xFF)
        g.launch()
        st.synchronize()
        assert np.array_equal(dD.to_host(), want)
    g.close()
    gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, 4, st.h)   # the stream's workspace
    st.synchronize()
    assert np.array_equal(dC.to_host(), want)
    with gpu.Graph(st) as g2:
        gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, 4, st.h)
        gpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dD.ptr, M, N, K, st.h)
    for _ in range(3):
        dC.fill_bytes(0xFF)
        dD.fill_bytes(0xFF)
        g2.launch()
        st.synchronize()
        assert np.array_equal(dC.to_host(), want) and np.array_equal(dD.to_host(), want)
    g2.close()
    st.close()


def test_splitk_graph_outlives_its_stream(gpu):
    """A graph recorded on a stream holds that stream's split-K workspace: after the stream is
    destroyed the graph still replays exactly (here on another stream, between that stream's
    own split launches); destroying the graph then frees it, and streams made afterwards
    (whose handles may repeat the destroyed one's) get workspaces of their own."""
    M, N, K = 768, 768, 2048                                # sgpu_sgemm_opt splits this one 5 ways
    rng = np.random.default_rng(29)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC, dD = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N)), \
        gpu.DeviceArray((M, N))
    st = gpu.Stream()
    gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, 4, st.h)   # the stream's workspace
    st.synchronize()
    with gpu.Graph(st) as g:
        gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, 4, st.h)
    st.close()                                              # the graph keeps its workspace
    st2 = gpu.Stream()
    for _ in range(3):
        dC.fill_bytes(0xFF)
        gpu.call("sgpu_graph_launch", g.h, st2.h)
        st2.synchronize()
        assert np.array_equal(dC.to_host(), want)
        dD.fill_bytes(0xFF)
        gpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dD.ptr, M, N, K, st2.h)   # st2's own workspace
        st2.synchronize()
        assert np.array_equal(dD.to_host(), want)
    g.close()
    for _ in range(2):
        st3 = gpu.Stream()
        dC.fill_bytes(0xFF)
        gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, 4, st3.h)
        st3.synchronize()
        assert np.array_equal(dC.to_host(), want)
        st3.close()
    st2.close()


def test_per_thread_stream_has_no_workspace(gpu):
    """hipStreamPerThread names a different stream in every host thread, so it gets no split-K
    workspace: sgpu_sgemm_splitk refuses it, sgpu_sgemm_opt runs its unsplit member there."""
    per_thread = ct.c_void_p(2)                             # hipStreamPerThread
    M, N, K = 768, 768, 2048
    rng = np.random.default_rng(31)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    assert gpu.lib().sgpu_sgemm_splitk(dA.ptr, dB.ptr, dC.ptr, M, N, K, 4, per_thread) == gpu.SGPU_ERR_NO_WORKSPACE
    dC.fill_bytes(0xFF)
    gpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, M, N, K, per_thread)
    gpu.call("sgpu_stream_synchronize", per_thread)
    assert np.array_equal(dC.to_host(), want)


def test_gemv_multi_workspace_only_when_split(gpu, og):
    """sgpu_gemv_multi makes a stream's split-K workspace (32 MB) only for a launch that splits:
    the few-token register GEMV allocates nothing on a new stream; a matrix-core launch with
    too few 32x32 tiles to fill the CUs makes it, once."""
    hip = ct.CDLL("libamdhip64.so")

    def free_bytes():
        f, t = ct.c_size_t(), ct.c_size_t()
        gpu.synchronize()
        assert hip.hipMemGetInfo(ct.byref(f), ct.byref(t)) == 0
        return f.value

    K, N = 768, 64
    W, s = gpu.gen_normal(N * K, 41, 0.0, 0.02)
    X, _ = gpu.gen_normal(32 * K, s, 0.0, 1.0)
    dW, dX, dY = gpu.DeviceArray.from_host(W), gpu.DeviceArray.from_host(X), gpu.DeviceArray((32, N))
    st = gpu.Stream()
    for T, grows in ((2, False), (8, False), (32, True), (32, False)):
        before = free_bytes()
        dY.fill_bytes(0xFF)
        gpu.call("sgpu_gemv_multi", dW.ptr, dX.ptr, None, dY.ptr, K, N, T, st.h)
        st.synchronize()
        used = before - free_bytes()
        say(f"gemv_multi T={T}: {used} bytes of device memory")
        assert (used >= 32 << 20) if grows else (used < 8 << 20), (T, used)
        ref = og.gemv_multi(W, X[:T * K], None, K, N, T).reshape(T, N)
        assert np.all(np.abs(dY.to_host()[:T] - ref) <= 1e-4 * np.abs(ref) + 1e-4)
    st.close()


SMALL_CASES = [(1, 1, 1), (16, 16, 16), (33, 17, 96), (7, 300, 13), (256, 256, 256), (512, 512, 512),
               (100, 70, 3000), (130, 260, 40), (257, 511, 1030), (1023, 1025, 997), (64, 48, 2)]


@pytest.mark.parametrize("tile", [16, 32])
@pytest.mark.parametrize("M,N,K", SMALL_CASES)
def test_small_integer_exact(gpu, M, N, K, tile):
    """The small-problem members give the exact product on integer inputs (K tails, partial
    tiles, K % 4 != 0 on the scalar A path), twice in a row."""
    say(f"sgemm small{tile} integer {M}x{N}x{K}")
    rng = np.random.default_rng(M * 3 + N * 5 + K + tile)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    for _ in range(2):
        dC.fill_bytes(0xFF)
        gpu.call("sgpu_sgemm_small", dA.ptr, dB.ptr, dC.ptr, M, N, K, tile, None)
        gpu.synchronize()
        assert np.array_equal(dC.to_host(), want)


# sgemm_kwave splits each tile's 16-deep slices over the block's four waves: two slices (two
# waves idle), six (uneven), one or two per wave (no pipelined pair, one pair), odd counts per
# wave (the pipeline's tail slice), and up to 64 slices per wave.
KWAVE_CASES = [(64, 64, 32), (64, 64, 96), (64, 128, 160), (128, 192, 1024), (256, 320, 544),
               (512, 1024, 2048), (64, 64, 4096), (1024, 1024, 1024), (64, 64, 64), (128, 64, 128),
               (64, 128, 192), (192, 64, 224), (64, 64, 352)]


@pytest.mark.parametrize("M,N,K", KWAVE_CASES)
def test_kwave_integer_exact(gpu, M, N, K):
    """sgemm_kwave gives the exact product on integer inputs, twice in a row."""
    say(f"sgemm kwave integer {M}x{N}x{K}")
    rng = np.random.default_rng(M * 13 + N * 7 + K)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    for _ in range(2):
        dC.fill_bytes(0xFF)
        gpu.call("sgpu_sgemm_kwave", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
        gpu.synchronize()
        assert np.array_equal(dC.to_host(), want)


def test_kwave_reference_inputs(gpu, og):
    """Reference-generator inputs at 1024^3 within the normwise bar of the oracle."""
    n = 1024
    say(f"sgemm kwave n={n} reference inputs")
    A, B = ref_inputs(n, n, n)
    C = run_sgemm(gpu, "sgpu_sgemm_kwave", A, B, n, n, n)
    ref = ref_golden(n, n, n)
    assert np.abs(C.astype(np.float64) - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    assert og.sgemm_verdict_bad(C, ref, n, n) == 0


def test_kwave_graph_replay(gpu):
    """sgemm_kwave recorded once in a graph and replayed with new inputs copied in between:
    every replay equals the direct launch bit for bit (it uses no workspace and no fills)."""
    M, N, K = 256, 512, 2048
    say(f"sgemm kwave graph replay {M}x{N}x{K}")
    dA, dB, dC, dD = gpu.DeviceArray((M, K)), gpu.DeviceArray((K, N)), gpu.DeviceArray((M, N)), gpu.DeviceArray((M, N))
    st = gpu.Stream()
    with gpu.Graph(st) as g:
        gpu.call("sgpu_sgemm_kwave", dA.ptr, dB.ptr, dC.ptr, M, N, K, st.h)
    for rep in range(4):
        rng = np.random.default_rng(500 + rep)
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((K, N)).astype(np.float32)
        gpu.call("sgpu_memcpy_htod", dA.ptr, A.ctypes.data, A.nbytes)
        gpu.call("sgpu_memcpy_htod", dB.ptr, B.ctypes.data, B.nbytes)
        gpu.call("sgpu_sgemm_kwave", dA.ptr, dB.ptr, dD.ptr, M, N, K, st.h)
        st.synchronize()
        dC.fill_bytes(0xFF)
        g.launch()
        st.synchronize()
        assert np.array_equal(dC.to_host().view(np.uint32), dD.to_host().view(np.uint32)), rep
        ref = A.astype(np.float64) @ B.astype(np.float64)
        assert np.abs(dC.to_host() - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    g.close()
    st.close()


def test_kwave_rejects_other_shapes(gpu):
    """Shapes sgemm_kwave does not take, and operands off 16-byte alignment, are refused
    before any launch; M or N = 0 is a no-op."""
    dA, dB, dC = gpu.DeviceArray(64 * 4096 + 4), gpu.DeviceArray(4096 * 128 + 4), gpu.DeviceArray(64 * 128)
    L = gpu.lib()
    for M, N, K in ((63, 64, 64), (64, 96, 64), (64, 64, 48), (64, 64, 0), (-64, 64, 64)):
        assert L.sgpu_sgemm_kwave(dA.ptr, dB.ptr, dC.ptr, M, N, K, None) == gpu.SGPU_ERR_INVALID_ARG, (M, N, K)
    assert L.sgpu_sgemm_kwave(dA.offset(1), dB.ptr, dC.ptr, 64, 64, 64, None) == gpu.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_kwave(dA.ptr, dB.offset(2), dC.ptr, 64, 64, 64, None) == gpu.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_kwave(dA.ptr, dB.ptr, dC.ptr, 0, 64, 64, None) == 0


def test_opt_unaligned_kwave_shape_takes_the_edge_member(gpu):
    """sgpu_sgemm_opt plans sgemm_kwave for 1024^3; with A off 16-byte alignment it launches
    sgemm_kwave_edge instead (rows of any float alignment), whose C it then equals bit for
    bit."""
    M = N = K = 1024
    A, B = ref_inputs(M, N, K)
    C = run_sgemm(gpu, "sgpu_sgemm_opt", A, B, M, N, K, a_off=1)
    D = run_sgemm(gpu, "sgpu_sgemm_kwave_edge", A, B, M, N, K, a_off=1)
    assert np.array_equal(C, D)


# sgemm_kwave_edge: M, N >= 64 with partial last rows and columns of tiles (computed as the 64
# ending at the last one), N % 64 == 1 (the column computed by the last column of whole tiles:
# one such column, many; with 16 or more tile columns it is spread over all of them, 4, 2 or
# 1 rows a tile, some tiles with none), K tails of 1..15 (the partial first slice: up to 8 deep, one lane half
# padded; 9..15, both halves partly real) and K < 16 (the partial slice alone), a wave holding
# only the partial slice, one slice (three waves idle), uneven quarters, up to 260 slices per
# wave, and rows of any float alignment.
EDGE_CASES = [(64, 64, 1), (64, 65, 37), (130, 64, 33), (127, 129, 131), (64, 64, 5), (200, 191, 3),
              (64, 127, 100), (100, 100, 2), (65, 4097, 64), (300, 1025, 2047), (64, 65, 4103),
              (1023, 1025, 997), (1024, 1024, 1000), (1023, 1000, 997), (8192, 128, 1000),
              (64, 64, 16), (64, 64, 17), (65, 66, 25), (128, 130, 47), (64, 129, 24), (64, 65, 25),
              (130, 1281, 100), (70, 2561, 33)]


@pytest.mark.parametrize("a_off,b_off", [(0, 0), (1, 3)])
@pytest.mark.parametrize("M,N,K", EDGE_CASES)
def test_kwave_edge_integer_exact(gpu, M, N, K, a_off, b_off):
    """sgemm_kwave_edge gives the exact product on integer inputs, twice in a row, with C
    pre-filled with NaN (an unwritten element shows) and A, B at any float offset."""
    say(f"sgemm kwave_edge integer {M}x{N}x{K} a_off={a_off} b_off={b_off}")
    rng = np.random.default_rng(M * 17 + N * 5 + K + a_off)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    for _ in range(2):
        assert np.array_equal(run_sgemm(gpu, "sgpu_sgemm_kwave_edge", A, B, M, N, K, a_off, b_off), want)


@pytest.mark.parametrize("M,N,K", [(1023, 1025, 997), (1000, 1000, 1000)])
def test_kwave_edge_reference_inputs(gpu, og, M, N, K):
    """Reference-generator inputs within the normwise bar of the oracle and its verdict clean,
    on the reference's ragged shape (one column past 16 whole tiles) and on clamped edge tiles."""
    say(f"sgemm kwave_edge {M}x{N}x{K} reference inputs")
    A, B = ref_inputs(M, N, K)
    C = run_sgemm(gpu, "sgpu_sgemm_kwave_edge", A, B, M, N, K)
    ref = ref_golden(M, N, K)
    assert np.abs(C.astype(np.float64) - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    assert og.sgemm_verdict_bad(C, ref, M, N) == 0


@pytest.mark.parametrize("a_off", [0, 1])
@pytest.mark.parametrize("M,N,K", [(100, 70, 3000), (257, 511, 1030), (64, 65, 37), (1023, 1025, 997)])
def test_kwave_edge_operands_followed_by_nan(gpu, M, N, K, a_off):
    """A and B at the start of larger NaN-filled allocations, as for the other members: the
    edge member's partial last slice, its clamped edge tiles and the extra column's loads
    read nothing past either operand."""
    say(f"sgemm kwave_edge nan-padded {M}x{N}x{K} a_off={a_off}")
    rng = np.random.default_rng(M * 5 + N * 3 + K + 1)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    ha = np.full(a_off + M * K + K + 512, np.nan, np.float32)
    ha[a_off:a_off + M * K] = A.reshape(-1)
    hb = np.full((K + 512) * N, np.nan, np.float32)
    hb[:K * N] = B.reshape(-1)
    dA, dB, dC = gpu.DeviceArray.from_host(ha), gpu.DeviceArray.from_host(hb), gpu.DeviceArray((M, N))
    for _ in range(2):
        dC.fill_bytes(0xFF)
        gpu.call("sgpu_sgemm_kwave_edge", dA.offset(a_off), dB.ptr, dC.ptr, M, N, K, None)
        gpu.synchronize()
        assert np.array_equal(dC.to_host(), want)


@pytest.mark.parametrize("last_col", [False, True])
@pytest.mark.parametrize("M,N,K", [(127, 129, 131), (64, 65, 37), (1023, 1025, 997), (1000, 1000, 1000)])
def test_kwave_edge_nonfinite_inputs_propagate(gpu, M, N, K, last_col):
    """The non-finite operands of the other members through sgemm_kwave_edge, the infinities
    in B's row K-1 (the partial last slice where K % 32 != 0) and row 0, in column N/2 or in
    column N-1 (with N % 64 == 1 the column the last whole tiles compute by VALU FMAs)."""
    say(f"sgemm kwave_edge non-finite {M}x{N}x{K} last_col={last_col}")
    A, B, want = nonfinite_operands(M, N, K, M + 7 * N + 3 * K, jb=N - 1 if last_col else None)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    dC.fill_bytes(0xFF)
    gpu.call("sgpu_sgemm_kwave_edge", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
    gpu.synchronize()
    got = dC.to_host()
    assert np.array_equal(got, want, equal_nan=True), (np.argwhere(~((got == want) | (np.isnan(got) & np.isnan(want))))[:5])


def test_kwave_edge_graph_replay(gpu):
    """sgemm_kwave_edge recorded once in a graph and replayed with new inputs copied in
    between: every replay equals the direct launch bit for bit."""
    M, N, K = 1023, 1025, 997
    say(f"sgemm kwave_edge graph replay {M}x{N}x{K}")
    dA, dB, dC, dD = gpu.DeviceArray((M, K)), gpu.DeviceArray((K, N)), gpu.DeviceArray((M, N)), gpu.DeviceArray((M, N))
    st = gpu.Stream()
    with gpu.Graph(st) as g:
        gpu.call("sgpu_sgemm_kwave_edge", dA.ptr, dB.ptr, dC.ptr, M, N, K, st.h)
    for rep in range(4):
        rng = np.random.default_rng(700 + rep)
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((K, N)).astype(np.float32)
        gpu.call("sgpu_memcpy_htod", dA.ptr, A.ctypes.data, A.nbytes)
        gpu.call("sgpu_memcpy_htod", dB.ptr, B.ctypes.data, B.nbytes)
        gpu.call("sgpu_sgemm_kwave_edge", dA.ptr, dB.ptr, dD.ptr, M, N, K, st.h)
        st.synchronize()
        dC.fill_bytes(0xFF)
        g.launch()
        st.synchronize()
        assert np.array_equal(dC.to_host().view(np.uint32), dD.to_host().view(np.uint32)), rep
        ref = A.astype(np.float64) @ B.astype(np.float64)
        assert np.abs(dC.to_host() - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    g.close()
    st.close()


def test_kwave_edge_rejects_other_shapes(gpu):
    """M or N below 64, K = 0, negative sizes, null or non-float-aligned operands are refused
    before any launch; M or N = 0 is a no-op."""
    dA, dB, dC = gpu.DeviceArray(64 * 4096 + 4), gpu.DeviceArray(4096 * 128 + 4), gpu.DeviceArray(64 * 128 + 4)
    L = gpu.lib()
    for M, N, K in ((63, 64, 64), (64, 63, 64), (64, 64, 0), (-64, 64, 64), (64, 64, -1)):
        assert L.sgpu_sgemm_kwave_edge(dA.ptr, dB.ptr, dC.ptr, M, N, K, None) == gpu.SGPU_ERR_INVALID_ARG, (M, N, K)
    assert L.sgpu_sgemm_kwave_edge(dA.ptr + 2, dB.ptr, dC.ptr, 64, 64, 64, None) == gpu.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_kwave_edge(dA.ptr, dB.ptr + 1, dC.ptr, 64, 64, 64, None) == gpu.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_kwave_edge(dA.ptr, dB.ptr, dC.ptr + 3, 64, 64, 64, None) == gpu.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_kwave_edge(None, dB.ptr, dC.ptr, 64, 64, 64, None) == gpu.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_kwave_edge(dA.ptr, dB.ptr, dC.ptr, 0, 64, 64, None) == 0
    assert L.sgpu_sgemm_kwave_edge(dA.ptr, dB.ptr, dC.ptr, 64, 0, 64, None) == 0


NAN_PAD_CASES = [(7, 300, 13), (100, 70, 3000), (33, 17, 96), (64, 48, 2), (257, 511, 1030)]


@pytest.mark.parametrize("a_off", [0, 1])
@pytest.mark.parametrize("launcher", ["small16", "small32", "splitk4", "sgpu_sgemm_opt", "sgpu_sgemm_tiled",
                                      "sgpu_sgemm_opt256"])
@pytest.mark.parametrize("M,N,K", NAN_PAD_CASES)
def test_operands_followed_by_nan_integer_exact(gpu, M, N, K, launcher, a_off):
    """A and B sit at the start of larger allocations whose remaining floats are NaN: 512 rows
    of B past row K-1 and K + 512 floats past A's last element (more than any load of a K tail
    or k-group batch reaches).  A kernel that read past either operand would put NaN into C
    (0 * NaN); every read stays inside the allocations, so the run is in bounds either way.
    a_off = 1 starts A one float past a 16-byte boundary (scalar A loads)."""
    say(f"sgemm {launcher} nan-padded {M}x{N}x{K} a_off={a_off}")
    rng = np.random.default_rng(M * 5 + N * 3 + K)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    ha = np.full(a_off + M * K + K + 512, np.nan, np.float32)
    ha[a_off:a_off + M * K] = A.reshape(-1)
    hb = np.full((K + 512) * N, np.nan, np.float32)
    hb[:K * N] = B.reshape(-1)
    dA, dB, dC = gpu.DeviceArray.from_host(ha), gpu.DeviceArray.from_host(hb), gpu.DeviceArray((M, N))
    for _ in range(2):
        dC.fill_bytes(0xFF)
        if launcher.startswith("small"):
            gpu.call("sgpu_sgemm_small", dA.offset(a_off), dB.ptr, dC.ptr, M, N, K, int(launcher[5:]), None)
        elif launcher == "splitk4":
            gpu.call("sgpu_sgemm_splitk", dA.offset(a_off), dB.ptr, dC.ptr, M, N, K, 4, None)
        else:
            gpu.call(launcher, dA.offset(a_off), dB.ptr, dC.ptr, M, N, K, None)
        gpu.synchronize()
        assert np.array_equal(dC.to_host(), want)


NONFINITE_CASES = [(7, 300, 13), (100, 70, 3000), (130, 190, 65), (256, 256, 256), (1023, 1025, 997)]


def nonfinite_operands(M, N, K, seed, jb=None):
    """Small integers plus: NaN at A[ia, ka]; +Inf at B[kb, jb] and -Inf at B[0, jb] (jb
    N // 2 unless given); a zero at A[iz, kb].  Returns A, B and the IEEE product the reference's serial fp32 loop
    (gpu_workload.c:97-98) yields: row ia all NaN (NaN times anything); in column jb,
    A[i,kb]*Inf + A[i,0]*(-Inf) is NaN when either multiplier is 0 (Inf * 0) or the two
    infinities have opposite signs, else that infinity; everything else the exact integer sum."""
    rng = np.random.default_rng(seed)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    ia, ka, kb, iz = M // 2, K // 3, K - 1, (M // 2 + 1) % M
    jb = N // 2 if jb is None else jb
    A[iz, kb] = 0.0
    Af, Bf = A.copy(), B.copy()
    A[ia, ka] = np.nan
    B[kb, jb], B[0, jb] = np.inf, -np.inf
    Bf[kb, jb] = Bf[0, jb] = 0.0
    want = (Af.astype(np.float64) @ Bf.astype(np.float64)).astype(np.float32)
    t1 = np.sign(A[:, kb])                 # sign of A[i,kb] * +Inf (0: NaN)
    t2 = -np.sign(A[:, 0])                 # sign of A[i,0] * -Inf (0: NaN)
    with np.errstate(invalid="ignore"):
        col = np.where((t1 == 0) | (t2 == 0) | (t1 != t2), np.nan, t1 * np.inf).astype(np.float32)
    want[:, jb] = col
    want[ia, :] = np.nan
    return A, B, want


@pytest.mark.parametrize("launcher", ["small16", "small32", "splitk4", "sgpu_sgemm_opt", "sgpu_sgemm_tiled",
                                      "sgpu_sgemm_tiled4", "sgpu_sgemm_opt256"])
@pytest.mark.parametrize("M,N,K", NONFINITE_CASES)
def test_nonfinite_inputs_propagate(gpu, M, N, K, launcher):
    """NaN and Inf inside A and B come out of every launch form as the reference's IEEE
    fp32 arithmetic has them (no path zeroes, clamps or skips an in-bounds element), and the
    finite elements stay exact."""
    say(f"sgemm {launcher} non-finite {M}x{N}x{K}")
    A, B, want = nonfinite_operands(M, N, K, M + 7 * N + 3 * K)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    dC.fill_bytes(0xFF)
    if launcher.startswith("small"):
        gpu.call("sgpu_sgemm_small", dA.ptr, dB.ptr, dC.ptr, M, N, K, int(launcher[5:]), None)
    elif launcher == "splitk4":
        gpu.call("sgpu_sgemm_splitk", dA.ptr, dB.ptr, dC.ptr, M, N, K, 4, None)
    else:
        gpu.call(launcher, dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
    gpu.synchronize()
    got = dC.to_host()
    assert np.array_equal(got, want, equal_nan=True), (np.argwhere(~((got == want) | (np.isnan(got) & np.isnan(want))))[:5])


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (128, 192, 1024), (1024, 1024, 1024)])
def test_kwave_nonfinite_inputs_propagate(gpu, M, N, K):
    """The same non-finite operands through sgemm_kwave (whole tiles, K a multiple of 32):
    the wave holding the NaN's or an infinity's k-quarter carries it into the tile's sum."""
    say(f"sgemm kwave non-finite {M}x{N}x{K}")
    A, B, want = nonfinite_operands(M, N, K, M + 7 * N + 3 * K)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    dC.fill_bytes(0xFF)
    gpu.call("sgpu_sgemm_kwave", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
    gpu.synchronize()
    got = dC.to_host()
    assert np.array_equal(got, want, equal_nan=True), (np.argwhere(~((got == want) | (np.isnan(got) & np.isnan(want))))[:5])


# sgemm_kwave128 hands each tile's 16-deep slices to the block's four waves in pairs: one pair
# (three waves idle), two and three pairs (uneven), one pair each, many pairs each, one tile,
# one round of tiles and a grid of several rounds (2304 x 2048: 288 tiles).
KWAVE128_CASES = [(128, 128, 32), (128, 128, 64), (128, 256, 96), (256, 128, 128), (384, 256, 352),
                  (128, 128, 4096), (1024, 1024, 1024), (2048, 2048, 256), (2304, 2048, 64)]


@pytest.mark.parametrize("M,N,K", KWAVE128_CASES)
def test_kwave128_integer_exact(gpu, M, N, K):
    """sgemm_kwave128 gives the exact product on integer inputs, twice in a row."""
    say(f"sgemm kwave128 integer {M}x{N}x{K}")
    rng = np.random.default_rng(M * 11 + N * 5 + K)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    for _ in range(2):
        dC.fill_bytes(0xFF)
        gpu.call("sgpu_sgemm_kwave128", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
        gpu.synchronize()
        assert np.array_equal(dC.to_host(), want)


def test_kwave128_reference_inputs(gpu, og):
    """Reference-generator inputs at 1024^3 within the normwise bar of the oracle."""
    n = 1024
    say(f"sgemm kwave128 n={n} reference inputs")
    A, B = ref_inputs(n, n, n)
    C = run_sgemm(gpu, "sgpu_sgemm_kwave128", A, B, n, n, n)
    ref = ref_golden(n, n, n)
    assert np.abs(C.astype(np.float64) - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    assert og.sgemm_verdict_bad(C, ref, n, n) == 0


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (384, 128, 1024)])
def test_kwave128_nonfinite_inputs_propagate(gpu, M, N, K):
    """The non-finite operands of the other members through sgemm_kwave128."""
    say(f"sgemm kwave128 non-finite {M}x{N}x{K}")
    A, B, want = nonfinite_operands(M, N, K, M + 5 * N + 3 * K)
    dA, dB, dC = gpu.DeviceArray.from_host(A), gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    dC.fill_bytes(0xFF)
    gpu.call("sgpu_sgemm_kwave128", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
    gpu.synchronize()
    got = dC.to_host()
    assert np.array_equal(got, want, equal_nan=True), (np.argwhere(~((got == want) | (np.isnan(got) & np.isnan(want))))[:5])


def test_kwave128_graph_replay(gpu):
    """sgemm_kwave128 recorded once in a graph and replayed with new inputs copied in between:
    every replay equals the direct launch bit for bit (it uses no workspace and no fills)."""
    M, N, K = 256, 384, 1024
    say(f"sgemm kwave128 graph replay {M}x{N}x{K}")
    dA, dB, dC, dD = gpu.DeviceArray((M, K)), gpu.DeviceArray((K, N)), gpu.DeviceArray((M, N)), gpu.DeviceArray((M, N))
    st = gpu.Stream()
    with gpu.Graph(st) as g:
        gpu.call("sgpu_sgemm_kwave128", dA.ptr, dB.ptr, dC.ptr, M, N, K, st.h)
    for rep in range(4):
        rng = np.random.default_rng(700 + rep)
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((K, N)).astype(np.float32)
        gpu.call("sgpu_memcpy_htod", dA.ptr, A.ctypes.data, A.nbytes)
        gpu.call("sgpu_memcpy_htod", dB.ptr, B.ctypes.data, B.nbytes)
        gpu.call("sgpu_sgemm_kwave128", dA.ptr, dB.ptr, dD.ptr, M, N, K, st.h)
        st.synchronize()
        dC.fill_bytes(0xFF)
        g.launch()
        st.synchronize()
        assert np.array_equal(dC.to_host().view(np.uint32), dD.to_host().view(np.uint32)), rep
        ref = A.astype(np.float64) @ B.astype(np.float64)
        assert np.abs(dC.to_host() - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    g.close()
    st.close()


def test_kwave128_rejects_other_shapes(gpu):
    """Shapes sgemm_kwave128 does not take (including a 128-row A panel or a 16-row B slice of
    2^31 bytes), and operands off 16-byte alignment, are refused before any launch; M or N = 0
    is a no-op."""
    dA, dB, dC = gpu.DeviceArray(128 * 4096 + 4), gpu.DeviceArray(4096 * 256 + 4), gpu.DeviceArray(128 * 256)
    L = gpu.lib()
    for M, N, K in ((64, 128, 64), (128, 192, 64), (128, 128, 48), (128, 128, 16), (128, 128, 0), (-128, 128, 64),
                    (128, 128, 1 << 22), (128, 1 << 25, 32)):
        assert L.sgpu_sgemm_kwave128(dA.ptr, dB.ptr, dC.ptr, M, N, K, None) == gpu.SGPU_ERR_INVALID_ARG, (M, N, K)
    assert L.sgpu_sgemm_kwave128(dA.offset(1), dB.ptr, dC.ptr, 128, 128, 64, None) == gpu.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_kwave128(dA.ptr, dB.offset(2), dC.ptr, 128, 128, 64, None) == gpu.SGPU_ERR_INVALID_ARG
    assert L.sgpu_sgemm_kwave128(dA.ptr, dB.ptr, dC.ptr, 0, 128, 64, None) == 0


def test_opt_unaligned_kwave128_shape_takes_the_size_rule_member(gpu):
    """sgpu_sgemm_opt plans sgemm_kwave128 for 2048^3; with A off 16-byte alignment it launches
    the member the size rule picks (sgemm_tiled4), whose C it then equals bit for bit."""
    M = N = K = 2048
    rng = np.random.default_rng(2048)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    C = run_sgemm(gpu, "sgpu_sgemm_opt", A, B, M, N, K, a_off=1)
    D = run_sgemm(gpu, "sgpu_sgemm_tiled4", A, B, M, N, K, a_off=1)
    assert np.array_equal(C, D)


@pytest.mark.parametrize("tile", [16, 32])
def test_small_reference_generator_unaligned_and_k_zero(gpu, og, tile):
    """Reference-generator inputs within the normwise bar of the oracle with A one float past
    a 16-byte boundary (scalar A path), and K = 0 writing zeros."""
    M, N, K = 200, 300, 512
    say(f"sgemm small{tile} srand unaligned {M}x{N}x{K}")
    A, B = gpu.gen_sgemm_inputs(max(M * K, K * N), 42)
    A, B = A[:M * K], B[:K * N]
    dA = gpu.DeviceArray(M * K + 1)
    gpu.call("sgpu_memcpy_htod", dA.offset(1), A.ctypes.data, M * K * 4)
    dB, dC = gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    gpu.call("sgpu_sgemm_small", dA.offset(1), dB.ptr, dC.ptr, M, N, K, tile, None)
    gpu.synchronize()
    C = dC.to_host().reshape(M, N)
    ref = og.sgemm(A, B, M, N, K).astype(np.float64)
    assert np.abs(C - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    dC.fill_bytes(0xFF)
    gpu.call("sgpu_sgemm_small", dA.ptr, dB.ptr, dC.ptr, 5, 7, 0, tile, None)
    gpu.synchronize()
    assert np.array_equal(dC.to_host().reshape(-1)[:35], np.zeros(35, np.float32))


def test_splitk_reference_generator_and_unaligned(gpu, og):
    """Reference-generator inputs within the normwise bar of the oracle, with A starting one
    float past a 16-byte boundary (every unit on the masked pipeline)."""
    M, N, K = 300, 200, 1500
    say(f"sgemm splitk srand unaligned {M}x{N}x{K}")
    A, B = gpu.gen_sgemm_inputs(max(M * K, K * N), 42)
    A, B = A[:M * K], B[:K * N]
    dA = gpu.DeviceArray(M * K + 1)
    gpu.call("sgpu_memcpy_htod", dA.offset(1), A.ctypes.data, M * K * 4)
    dB, dC = gpu.DeviceArray.from_host(B), gpu.DeviceArray((M, N))
    gpu.call("sgpu_sgemm_splitk", dA.offset(1), dB.ptr, dC.ptr, M, N, K, 6, None)
    gpu.synchronize()
    C = dC.to_host().reshape(M, N)
    ref = og.sgemm(A, B, M, N, K).astype(np.float64)
    assert np.abs(C - ref).max() / np.abs(ref).max() <= 1e-4


@pytest.mark.parametrize("fn", VARIANTS[:3] + ["sgpu_sgemm_opt256"])
def test_unaligned_pointers(gpu, fn):
    M, N, K = 200, 136, 72
    rng = np.random.default_rng(4)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    C = run_sgemm(gpu, fn, A, B, M, N, K, a_off=1, b_off=3)
    assert np.array_equal(C, (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("fn", VARIANTS)
def test_k_zero_writes_zeros_and_empty_is_noop(gpu, fn):
    C = run_sgemm(gpu, fn, np.zeros((5, 0), np.float32), np.zeros((0, 7), np.float32), 5, 7, 0)
    assert np.array_equal(C, np.zeros((5, 7), np.float32))
    assert getattr(gpu.lib(), fn)(None, None, None, 0, 7, 3, None) == 0


@pytest.mark.parametrize("n", [2048, 4096])
@pytest.mark.parametrize("fn", ["sgpu_sgemm_tiled4", "sgpu_sgemm_opt", "sgpu_sgemm_opt256"])
def test_full_size_integer_exact(gpu, fn, n):
    say(f"sgemm {fn} integer {n}^3")
    rng = np.random.default_rng(n)
    A = rng.integers(-2, 3, (n, n)).astype(np.float32)
    B = rng.integers(-2, 3, (n, n)).astype(np.float32)
    C = run_sgemm(gpu, fn, A, B, n, n, n)
    want = A.astype(np.float64) @ B.astype(np.float64)      # exact: |C| <= 4n < 2^24
    assert np.array_equal(C, want.astype(np.float32))


@pytest.mark.parametrize("n", [2048, 4096])
@pytest.mark.parametrize("fn", ["sgpu_sgemm_tiled", "sgpu_sgemm_tiled4", "sgpu_sgemm_opt"])
def test_full_size_reference_generator_sampled_rows(gpu, og, fn, n):
    """The sweep's 2048^3 and 4096^3 on the reference generator's inputs: 24 rows spread over
    C against the oracle's serial golden, normwise <= 1e-4 and the 5% verdict clean."""
    say(f"sgemm {fn} {n}^3 reference inputs, sampled rows")
    A, B = ref_inputs(n, n, n)
    C = run_sgemm(gpu, fn, A, B, n, n, n)
    rows = np.linspace(0, n - 1, 24).astype(int)
    ref = np.stack([og.sgemm_rows(A, B, n, n, n, r, r + 1, 1)[r] for r in rows])
    got = C[rows]
    assert np.abs(got.astype(np.float64) - ref).max() / np.abs(ref).max() <= NORMWISE_TOL
    assert og.sgemm_verdict_bad(got, ref, len(rows), n) == 0


@pytest.mark.parametrize("extra", [[], ["--ref-geometry"]])
def test_gpu_workload_harness_json(gpu, extra):
    """The harness flow end to end (module loaded from the .co file by path, kernels resolved
    by name): the --json object passes the task-queue consumer's checks
    (deploy/cluster/gpu_task_example.py:57-78) apart from its Tegra-sized GFLOPS bounds."""
    co = os.path.join(ROOT, "switch-l4t-gpu_amd", "build", "switch_gpu.co")
    cmd = [os.path.join(BIN, "gpu_workload"), "--json", "--membw-mb", "512", "--membw-iters", "2"] + extra
    if not extra:
        cmd += ["--extra", "2048", "--ragged"]
    say("run", " ".join(cmd))
    out = subprocess.run(cmd + [co], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    d = json.loads(out.stdout)
    assert d["done"] is True
    assert d["kernels"] == {"sgemm": "CORRECT", "sgemm_naive": "CORRECT", "sgemm_tiled4": "CORRECT",
                            "sgemm_opt": "CORRECT"}
    for key in ("sgemm", "sgemm4", "sgemm_opt"):
        assert [r["n"] for r in d[key]] == [256, 512, 1024]
        assert all(r["gflops"] > 1.0 for r in d[key])
    assert d["membw_gbps"] > 100.0
    for r in d.get("sgemm_extra", []):
        assert r["verdict"] == "CORRECT"
