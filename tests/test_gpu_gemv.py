"""Batch-1 GEMV family and the read-bandwidth probe on the GPU through the C ABI, against
the oracle (og_gemv: gemv_test.c:85-90 / gpt2_engine.c:342-349; og_gemv_h: qwen_engine.c:276-284;
og_gemv_multi: gpt2_kernels.cu:110-155 semantics; og_gemv_hh: the fp16-x form of gemv_h) and
exact integer arithmetic.

Bars: fp32 weights, per element |y - y_ref| <= 1e-4 |y_ref| + 1e-4 (gemv_test.c:119);
fp16 weights (fp32 accumulate) max|y - y_ref| / max|y_ref| <= 1e-3 and per element
1e-3 |y_ref| + 1e-3 max|y_ref|; integer-valued inputs bit-exact at every shape."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NT = min(16, os.cpu_count() or 1)
F32_KERNELS = ["sgpu_gemv", "sgpu_gemv4", "sgpu_gemv_warp"]
GPT2_SHAPES = [(2304, 768), (768, 768), (3072, 768), (768, 3072), (50257, 768)]      # [N x K]
QWEN_SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896), (1152, 896), (9728, 896)]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def gemv_dev(gpu, fn, W, x, bias, K, N, x_off=0):
    dW = gpu.DeviceArray.from_host(W)
    dx = gpu.DeviceArray(K + x_off + 1)
    gpu.call("sgpu_memcpy_htod", dx.offset(x_off), np.ascontiguousarray(x, np.float32).ctypes.data, K * 4)
    dy = gpu.DeviceArray(N)
    dy.fill_bytes(0xFF)
    db = gpu.DeviceArray.from_host(np.asarray(bias, np.float32)) if bias is not None else None
    if fn in F32_KERNELS:
        gpu.call(fn, dW.ptr, dx.offset(x_off), dy.ptr, K, N, None)
    else:
        gpu.call(fn, dW.ptr, dx.offset(x_off), db.ptr if db is not None else None, dy.ptr, K, N, None)
    gpu.synchronize()
    return dy.to_host()


@pytest.mark.parametrize("N,K", GPT2_SHAPES)
@pytest.mark.parametrize("fn", F32_KERNELS + ["sgpu_gemv_warp_b"])
def test_gpt2_shapes_fp32(gpu, og, fn, N, K):
    say(f"gemv {fn} {N}x{K}")
    W, s = gpu.gen_normal(N * K, 42 + N, 0.0, 0.02)
    x, s = gpu.gen_normal(K, s, 0.0, 1.0)
    bias = gpu.gen_normal(N, s, 0.0, 0.1)[0] if fn == "sgpu_gemv_warp_b" else None
    y = gemv_dev(gpu, fn, W, x, bias, K, N)
    ref = og.gemv(W, x, bias, K, N, NT)
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref) + 1e-4), np.abs(y - ref).max()


@pytest.mark.parametrize("N,K", QWEN_SHAPES)
def test_qwen_shapes_fp16(gpu, og, N, K):
    say(f"gemv_h {N}x{K}")
    Wf, s = gpu.gen_normal(N * K, 7 + N, 0.0, 0.02)
    W = gpu.f32_to_f16(Wf)
    x, s = gpu.gen_normal(K, s, 0.0, 1.0)
    bias = gpu.gen_normal(N, s, 0.0, 0.02)[0] if N == 1152 else None      # fused qkv carries a bias
    y = gemv_dev(gpu, "sgpu_gemv_h", W, x, bias, K, N)
    ref = og.gemv_h_fbias(W, x, bias, K, N, NT)
    m = np.abs(ref).max()
    assert np.abs(y - ref).max() / m <= 1e-3
    assert np.all(np.abs(y - ref) <= 1e-3 * np.abs(ref) + 1e-3 * m)


def gemv_hh_dev(gpu, W, x16, bias, K, N, x_off=0):
    """sgpu_gemv_hh with x (fp16 codes) placed x_off codes into its allocation."""
    dW = gpu.DeviceArray.from_host(W)
    dx = gpu.DeviceArray(K + x_off + 8, np.uint16)
    gpu.call("sgpu_memcpy_htod", dx.offset(x_off), np.ascontiguousarray(x16, np.uint16).ctypes.data, K * 2)
    dy = gpu.DeviceArray(N)
    dy.fill_bytes(0xFF)
    db = gpu.DeviceArray.from_host(np.asarray(bias, np.float32)) if bias is not None else None
    gpu.call("sgpu_gemv_hh", dW.ptr, dx.offset(x_off), db.ptr if db is not None else None, dy.ptr, K, N, None)
    gpu.synchronize()
    return dy.to_host()


@pytest.mark.parametrize("N,K", QWEN_SHAPES)
def test_qwen_shapes_fp16_x(gpu, og, N, K):
    """The fp16-x GEMV at every Qwen shape (fused qkv with its bias, gate|up, the lm_head):
    within the fp16 bars of the oracle, and bit for bit sgpu_gemv_h on the h2f-decoded x."""
    say(f"gemv_hh {N}x{K}")
    Wf, s = gpu.gen_normal(N * K, 11 + N, 0.0, 0.02)
    W = gpu.f32_to_f16(Wf)
    xf, s = gpu.gen_normal(K, s, 0.0, 1.0)
    x16 = gpu.f32_to_f16(xf)
    bias = gpu.gen_normal(N, s, 0.0, 0.02)[0] if N == 1152 else None
    y = gemv_hh_dev(gpu, W, x16, bias, K, N)
    ref = og.gemv_hh(W, x16, bias, K, N, NT)
    m = np.abs(ref).max()
    assert np.abs(y - ref).max() / m <= 1e-3
    assert np.all(np.abs(y - ref) <= 1e-3 * np.abs(ref) + 1e-3 * m)
    yh = gemv_dev(gpu, "sgpu_gemv_h", W, og.h2f_array(x16), bias, K, N)
    assert np.array_equal(y.view(np.uint32), yh.view(np.uint32))


EDGE_HH = [(1, 1), (5, 3), (64, 8), (63, 16), (1000, 63), (7, 896), (300, 4864), (33, 5000), (2, 40000)]


@pytest.mark.parametrize("N,K", EDGE_HH)
def test_gemv_hh_integer_exact_edges(gpu, N, K):
    """Integer-valued fp16 W, x and bias: exact at ragged K, with x aligned (tuned kernels)
    and one code off 16 bytes (the by-name gemv_hh symbol)."""
    say(f"gemv_hh integer {N}x{K}")
    rng = np.random.default_rng(N * 17 + K)
    Wi, xi, bi = rng.integers(-3, 4, (N, K)), rng.integers(-3, 4, K), rng.integers(-5, 6, N)
    W, x16 = Wi.astype(np.float16).view(np.uint16), xi.astype(np.float16).view(np.uint16)
    want = (Wi @ xi + bi).astype(np.float32)
    for x_off in (0, 1):
        assert np.array_equal(gemv_hh_dev(gpu, W, x16, bi, K, N, x_off=x_off), want)


def test_gemv_hh_special_x_codes(gpu, og):
    """x codes decoded with the reference h2f on the device: subnormals and -0 read +0,
    exponent-31 codes the finite 2^16 (1 + m/1024).  Integer W codes and at most 48
    exponent-31 x codes per row keep every fp32 partial sum exact (multiples of 64 below
    2^24 plus small integers), so the result is order-free and compared bit for bit."""
    rng = np.random.default_rng(23)
    N, K = 64, 896
    big = np.concatenate([np.arange(0x7c00, 0x8000), np.arange(0xfc00, 0x10000)]).astype(np.uint16)
    small = np.concatenate([np.arange(0, 1024), np.arange(0x8000, 0x8400),               # subnormals, -0
                            np.array([0x3c00, 0x4000, 0x4200, 0xbc00, 0xc000, 0xc200] * 50)]).astype(np.uint16)
    x16 = rng.choice(small, K).astype(np.uint16)
    x16[rng.choice(K, 48, replace=False)] = rng.choice(big, 48)
    W = rng.integers(-2, 3, (N, K)).astype(np.float16).view(np.uint16)
    ref = og.gemv_hh(W, x16, None, K, N)
    # independent of the oracle: the closed-form decode of x in float64
    e, m = (x16 >> 10) & 31, (x16 & 1023).astype(np.float64)
    sgn = np.where(x16 >> 15, -1.0, 1.0)
    xd = np.where(e == 0, 0.0, np.where(e == 31, sgn * 65536.0 * (1 + m / 1024), x16.view(np.float16).astype(np.float64)))
    assert np.array_equal(ref, (W.view(np.float16).astype(np.float64) @ xd).astype(np.float32))
    for x_off in (0, 1):
        assert np.array_equal(gemv_hh_dev(gpu, W, x16, None, K, N, x_off=x_off), ref)


def test_recorded_launches_replay(gpu, og):
    """GEMV (fp16 and fp32 weights) and SGEMM launches recorded once on a stream and replayed:
    every replay, with new inputs copied in between (host work and synchronisation between
    the replays), gives the same bits as the same launches run directly on that stream (whose
    split-K workspace was made before recording, so both take the split kernel)."""
    say("graph replay gemv_h + gemv_warp_b + sgemm_opt")
    N, K, M = 896, 4864, 64
    Wh = gpu.f32_to_f16(gpu.gen_normal(N * K, 3, 0.0, 0.02)[0])
    Wf, s = gpu.gen_normal(N * K, 5, 0.0, 0.02)
    bias, s = gpu.gen_normal(N, s, 0.0, 0.1)
    A, s = gpu.gen_normal(M * K, s, 0.0, 1.0)
    dWh, dWf, db, dA = (gpu.DeviceArray.from_host(a) for a in (Wh, Wf, bias, A))
    dx, dyh, dyf, dC = gpu.DeviceArray(K), gpu.DeviceArray(N), gpu.DeviceArray(N), gpu.DeviceArray((M, N))

    def launches(st):
        gpu.call("sgpu_gemv_h", dWh.ptr, dx.ptr, None, dyh.ptr, K, N, st)
        gpu.call("sgpu_gemv_warp_b", dWf.ptr, dx.ptr, db.ptr, dyf.ptr, K, N, st)
        # C[M x N] = A[M x K] * Wf viewed as [K x N]
        gpu.call("sgpu_sgemm_opt", dA.ptr, dWf.ptr, dC.ptr, M, N, K, st)

    st = gpu.Stream()
    launches(st.h)                  # the stream's split-K workspace exists before recording
    st.synchronize()
    with gpu.Graph(st) as g:
        launches(st.h)
    for rep in range(4):
        x, s = gpu.gen_normal(K, 100 + rep, 0.0, 1.0)
        gpu.call("sgpu_memcpy_htod", dx.ptr, x.ctypes.data, K * 4)
        for d in (dyh, dyf, dC):
            d.fill_bytes(0xFF)
        launches(st.h)              # the same launches on the same stream, run directly
        st.synchronize()
        want = [d.to_host() for d in (dyh, dyf, dC)]
        for d in (dyh, dyf, dC):
            d.fill_bytes(0xFF)
        g.launch()
        st.synchronize()
        got = [d.to_host() for d in (dyh, dyf, dC)]
        for w, h in zip(want, got):
            assert np.array_equal(w.view(np.uint32), h.view(np.uint32)), rep
        ref = og.gemv_h_fbias(Wh, x, None, K, N, NT)
        assert np.abs(got[0] - ref).max() / np.abs(ref).max() <= 1e-3
    g.close()
    st.close()


EDGE = [(1, 1), (5, 3), (64, 4), (63, 8), (1000, 63), (7, 896), (300, 4864), (33, 5000), (4, 8200), (2, 40000)]


@pytest.mark.parametrize("N,K", EDGE)
@pytest.mark.parametrize("fn", ["sgpu_gemv", "sgpu_gemv_warp_b", "sgpu_gemv_h"])
def test_integer_exact_edges(gpu, fn, N, K):
    say(f"gemv {fn} integer {N}x{K}")
    rng = np.random.default_rng(N * 13 + K)
    Wi = rng.integers(-3, 4, (N, K))
    xi = rng.integers(-3, 4, K)
    bi = rng.integers(-5, 6, N) if fn != "sgpu_gemv" else None
    W = Wi.astype(np.float16).view(np.uint16) if fn == "sgpu_gemv_h" else Wi.astype(np.float32)
    want = Wi @ xi + (bi if bi is not None else 0)
    for x_off in (0, 1):                                  # aligned and unaligned x
        y = gemv_dev(gpu, fn, W, xi.astype(np.float32), bi, K, N, x_off=x_off)
        assert np.array_equal(y, want.astype(np.float32))


def test_gemv_h_special_codes(gpu, og):
    """Subnormal and -0 codes read as +0, exponent-31 codes as 2^16 (1 + m/1024): the
    reference h2f contract (qwen_kernels.cu:6-14), exact with integer x."""
    rng = np.random.default_rng(3)
    N, K = 40, 896
    # subnormals, -0/negative subnormals, exponent 31 (values 65536 + 64m: integers), and
    # integer-valued normal codes 1, 2, 3, -1, -2 so every partial sum stays an exact fp32 integer
    codes = np.concatenate([np.arange(0, 1024), np.arange(0x8000, 0x8400), np.arange(0x7c00, 0x8000),
                            np.arange(0xfc00, 0x10000),
                            np.array([0x3c00, 0x4000, 0x4200, 0xbc00, 0xc000] * 40)]).astype(np.uint16)
    W = rng.choice(codes, (N, K)).astype(np.uint16)
    x = rng.integers(-2, 3, K).astype(np.float32)
    y = gemv_dev(gpu, "sgpu_gemv_h", W, x, None, K, N)
    assert np.array_equal(y, og.gemv_h(W, x, None, K, N))    # all terms are integers: order-free


@pytest.mark.parametrize("T", [1, 7, 16, 17, 128])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemv_multi(gpu, og, T, with_bias):
    say(f"gemv_multi T={T} bias={with_bias}")
    K, N = 768, 2304
    W, s = gpu.gen_normal(N * K, 5, 0.0, 0.02)
    X, s = gpu.gen_normal(T * K, s, 0.0, 1.0)
    bias = gpu.gen_normal(N, s, 0.0, 0.1)[0] if with_bias else None
    dW, dX = gpu.DeviceArray.from_host(W), gpu.DeviceArray.from_host(X)
    db = gpu.DeviceArray.from_host(bias) if with_bias else None
    dY = gpu.DeviceArray((T, N))
    dY.fill_bytes(0xFF)
    gpu.call("sgpu_gemv_multi", dW.ptr, dX.ptr, db.ptr if db else None, dY.ptr, K, N, T, None)
    gpu.synchronize()
    ref = og.gemv_multi(W, X, bias, K, N, T, NT)
    Y = dY.to_host()
    assert np.all(np.abs(Y - ref) <= 1e-4 * np.abs(ref) + 1e-4)


# (K, N, T): matrix-core path (32-token x 32-row tiles) with ragged token/row tiles, K tails
# inside a 32-deep chunk, K shorter than the four-wave split, the GPT-2 shapes, shapes with
# fewer tiles than CUs, whose tiles' K is split across blocks (the launcher's rule: up to 16
# splits of at least four 32-deep chunks), and up to 8 tokens on aligned rows, which take the
# register team GEMV (a wave per row to K = 1024, a block per row to K = 4096; beyond, the
# split matrix-core path).
MULTI_SHAPES = [(768, 2304, 128), (772, 100, 33), (64, 65, 1), (3072, 768, 64), (40, 1000, 300),
                (768, 2048, 512), (36, 37, 31), (768, 50257, 3), (4, 7, 5), (3072, 3072, 257),
                (64, 100, 3), (64, 100, 4), (1028, 40, 8), (1028, 40, 9), (1024, 40, 8),
                (4096, 96, 8), (4100, 96, 8), (3072, 768, 2)]


@pytest.mark.parametrize("K,N,T", MULTI_SHAPES)
def test_gemv_multi_integer_shapes(gpu, K, N, T):
    say(f"gemv_multi integer K={K} N={N} T={T}")
    rng = np.random.default_rng(K * 7 + N * 3 + T)
    W = rng.integers(-3, 4, (N, K))
    X = rng.integers(-3, 4, (T, K))
    bias = rng.integers(-50, 51, N).astype(np.float32)
    dW, dX = gpu.DeviceArray.from_host(W.astype(np.float32)), gpu.DeviceArray.from_host(X.astype(np.float32))
    db = gpu.DeviceArray.from_host(bias)
    dY = gpu.DeviceArray((T, N))
    dY.fill_bytes(0xFF)
    want = (X @ W.T + bias.astype(np.int64)).astype(np.float32)    # |sum| < 2^24: exact
    for _ in range(2):                         # split tiles leave their counters at zero
        dY.fill_bytes(0xFF)
        gpu.call("sgpu_gemv_multi", dW.ptr, dX.ptr, db.ptr, dY.ptr, K, N, T, None)
        gpu.synchronize()
        assert np.array_equal(dY.to_host(), want)


def test_gemv_multi_unaligned_rows_take_vector_path(gpu):
    rng = np.random.default_rng(8)
    K, N, T = 64, 96, 40
    W = rng.integers(-3, 4, (N, K)).astype(np.float32)
    X = rng.integers(-3, 4, (T, K)).astype(np.float32)
    dW = gpu.DeviceArray(N * K + 1)
    gpu.call("sgpu_memcpy_htod", dW.offset(1), W.ctypes.data, W.nbytes)
    dX = gpu.DeviceArray.from_host(X)
    dY = gpu.DeviceArray((T, N))
    gpu.call("sgpu_gemv_multi", dW.offset(1), dX.ptr, None, dY.ptr, K, N, T, None)
    gpu.synchronize()
    assert np.array_equal(dY.to_host(), (X.astype(np.float64) @ W.T.astype(np.float64)).astype(np.float32))


def test_gemv_multi_integer_ragged(gpu):
    rng = np.random.default_rng(6)
    K, N, T = 37, 29, 21
    W = rng.integers(-3, 4, (N, K))
    X = rng.integers(-3, 4, (T, K))
    dW, dX = gpu.DeviceArray.from_host(W.astype(np.float32)), gpu.DeviceArray.from_host(X.astype(np.float32))
    dY = gpu.DeviceArray((T, N))
    gpu.call("sgpu_gemv_multi", dW.ptr, dX.ptr, None, dY.ptr, K, N, T, None)
    gpu.synchronize()
    assert np.array_equal(dY.to_host(), (X @ W.T).astype(np.float32))


@pytest.mark.parametrize("groups,extra", [(3, 17), (19, 5), (16, 0)])
def test_membw_read4_sums(gpu, groups, extra):
    """Every thread's grid-stride sum, repeated `iters` times, lands in out[first index]
    (switch_gpu.cu:41-54); integer-valued data makes the sums exact.  Buffer sizes cover
    the tail loop only, the pipelined groups of eight plus a tail, and whole groups."""
    import ctypes as ct

    threads = ct.c_int()
    gpu.call("sgpu_membw_read4", None, None, 0, 1, ct.byref(threads), None)
    nthr = threads.value
    n4 = groups * nthr + extra
    rng = np.random.default_rng(8)
    buf = rng.integers(-8, 9, (n4, 4)).astype(np.float32)
    dbuf = gpu.DeviceArray.from_host(buf)
    dout = gpu.DeviceArray(nthr)
    dout.fill_bytes(0xFF)
    iters = 3
    gpu.call("sgpu_membw_read4", dbuf.ptr, dout.ptr, n4, iters, ct.byref(threads), None)
    gpu.synchronize()
    out = dout.to_host()
    row = buf.sum(axis=1)
    want = np.zeros(nthr)
    for j in range(0, n4, nthr):
        seg = row[j:j + nthr]
        want[:seg.size] += seg
    assert np.array_equal(out, (iters * want).astype(np.float32))


# ---- NaN / Inf inside the operands: IEEE propagation as the reference's serial loop has it ----
def _nonfinite(rows, cols, K, seed):
    """A (rows x K) with a NaN in row rows//2 and a 0 at [rows//2 + 1, K-1]; B (K x cols) with
    +Inf at [K-1, cols//2] and -Inf at [0, cols//2]; and the product the reference's serial
    fp32 loops give (gemv_test.c:85-90): the NaN row all NaN, in column cols//2
    A[i,K-1]*Inf + A[i,0]*(-Inf) is NaN when a multiplier is 0 or the infinities' signs differ,
    else that infinity; the rest the exact integer sum."""
    rng = np.random.default_rng(seed)
    A = rng.integers(-2, 3, (rows, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, cols)).astype(np.float32)
    ia, kb, jb, iz = rows // 2, K - 1, cols // 2, (rows // 2 + 1) % rows
    A[iz, kb] = 0.0
    Af, Bf = A.copy(), B.copy()
    A[ia, K // 3] = np.nan
    B[kb, jb], B[0, jb] = np.inf, -np.inf
    Bf[kb, jb] = Bf[0, jb] = 0.0
    want = (Af.astype(np.float64) @ Bf.astype(np.float64)).astype(np.float32)
    t1, t2 = np.sign(A[:, kb]), -np.sign(A[:, 0])
    with np.errstate(invalid="ignore"):
        want[:, jb] = np.where((t1 == 0) | (t2 == 0) | (t1 != t2), np.nan, t1 * np.inf)
    want[ia, :] = np.nan
    return A, B, want


@pytest.mark.parametrize("N,K", [(2304, 768), (768, 3072), (1000, 997)])
@pytest.mark.parametrize("fn,x_off", [("sgpu_gemv", 0), ("sgpu_gemv_warp_b", 0), ("sgpu_gemv_warp_b", 1)])
def test_fp32_gemv_nonfinite_propagate(gpu, fn, x_off, N, K):
    """NaN in a weight row and +-Inf in x come out of the team and the wave-per-row GEMVs
    (x_off = 1: unaligned x) as IEEE arithmetic has them; the finite rows stay exact."""
    say(f"gemv non-finite {fn} x_off={x_off} {N}x{K}")
    W, xcol, want = _nonfinite(N, 1, K, N + K + x_off)
    got = gemv_dev(gpu, fn, W, xcol[:, 0], None, K, N, x_off)
    assert np.array_equal(got, want[:, 0], equal_nan=True)


@pytest.mark.parametrize("K,N,T", [(768, 2304, 3), (768, 2304, 8), (768, 3072, 20), (3072, 768, 64), (997, 300, 5)])
def test_gemv_multi_nonfinite_propagate(gpu, K, N, T):
    """The batched GEMV (register, matrix-core, split and vector forms): a NaN weight row is NaN
    for every token; +-Inf in one token's X row reaches only that token's outputs."""
    say(f"gemv_multi non-finite K={K} N={N} T={T}")
    W, XT, want = _nonfinite(N, T, K, K + N + T)
    dW = gpu.DeviceArray.from_host(W)
    dX = gpu.DeviceArray.from_host(np.ascontiguousarray(XT.T))
    dY = gpu.DeviceArray((T, N))
    for _ in range(2):
        dY.fill_bytes(0xFF)
        gpu.call("sgpu_gemv_multi", dW.ptr, dX.ptr, None, dY.ptr, K, N, T, None)
        gpu.synchronize()
        assert np.array_equal(dY.to_host(), want.T, equal_nan=True)
