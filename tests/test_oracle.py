"""Pins the oracle (oracle/golden.c) against what fixes each function independently:
closed forms, exact integer arithmetic, library routines and the committed fixtures.
CPU only.  A plausible mistake in the restatement (a transposed operand, a dropped bias, a
wrong h2f branch, an off-by-one stride) fails at least one test here."""
import json
import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- h2f (qwen_engine.c:90-98)
def h2f_closed_form(codes):
    """Exponent 0 -> +0.0, 1..30 -> IEEE half (numpy's conversion), 31 -> (-1)^s 2^16 (1 + m/1024)."""
    codes = np.asarray(codes, np.uint16)
    e = (codes >> 10) & 31
    m = (codes & 1023).astype(np.float64)
    s = np.where(codes >> 15, -1.0, 1.0)
    out = codes.view(np.float16).astype(np.float32)
    out = np.where(e == 0, np.float32(0.0), out)
    out = np.where(e == 31, (s * 65536.0 * (1.0 + m / 1024.0)).astype(np.float32), out)
    return out.astype(np.float32)


def test_h2f_exhaustive(og):
    codes = np.arange(65536, dtype=np.uint16)
    got = og.h2f_array(codes)
    want = h2f_closed_form(codes)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # exponent-0 codes (subnormals and -0) give +0.0 exactly: sign dropped
    assert np.all(got[(codes >> 10) & 31 == 0].view(np.uint32) == 0)


def test_product_host_h2f_matches_oracle(og, sg):
    codes = np.arange(65536, dtype=np.uint16)
    prod = np.array([sg.lib().sgpu_h2f_host(int(c)) for c in codes], np.float32)
    assert np.array_equal(prod.view(np.uint32), og.h2f_array(codes).view(np.uint32))


# ------------------------------------------------------------- SGEMM (gpu_workload.c:97-98)
SHAPES = [(1, 1, 1), (7, 13, 5), (33, 65, 17), (64, 64, 64), (31, 17, 129), (5, 3, 0)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_sgemm_small_integers_exact(og, M, N, K):
    rng = np.random.default_rng(M * 1000 + N * 10 + K)
    A = rng.integers(-2, 3, size=(M, K))
    B = rng.integers(-2, 3, size=(K, N))
    C = og.sgemm(A, B, M, N, K)
    assert C.shape == (M, N)
    assert np.array_equal(C.astype(np.int64), A @ B)     # exact: |partial sums| < 2^24


def test_sgemm_identity_bitwise(og):
    rng = np.random.default_rng(1)
    B = rng.standard_normal((48, 40)).astype(np.float32)
    C = og.sgemm(np.eye(48, dtype=np.float32), B, 48, 40, 48)
    assert np.array_equal(C.view(np.uint32), B.view(np.uint32))


def test_sgemm_fp64_bound(og):
    """Serial fp32 summation error is at most K*eps*sum|a||b| (gamma_K bound)."""
    rng = np.random.default_rng(2)
    M, N, K = 40, 50, 300
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C = og.sgemm(A, B, M, N, K).astype(np.float64)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    bound = K * np.finfo(np.float32).eps * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    assert np.all(np.abs(C - ref) <= bound)


def test_sgemm_serial_order(og):
    """Pins the k-ascending serial order bit for bit on a case where order changes the result."""
    K = 4
    A = np.array([[1.0, 1e8, -1e8, 1.0]], np.float32)
    B = np.ones((K, 1), np.float32)
    # ((((0+1)+1e8)-1e8)+1) in fp32 = 1.0 ; any other order gives 0, 1 or 2
    assert og.sgemm(A, B, 1, 1, K)[0, 0] == np.float32(1.0)


def test_sgemm_rows_threaded_bitwise(og):
    rng = np.random.default_rng(3)
    M, N, K = 37, 29, 211
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    full = og.sgemm(A, B, M, N, K)
    part = og.sgemm_rows(A, B, M, N, K, 5, 30, nthreads=4)
    assert np.array_equal(part[5:30].view(np.uint32), full[5:30].view(np.uint32))
    assert np.isnan(part[:5]).all() and np.isnan(part[30:]).all()


def test_sgemm_verdict_predicate(og):
    """gpu_workload.c:101: |d| > 0.05|ref| + 1e-3 is bad, one count per row, stop at 5 rows."""
    ref = np.full((8, 8), 10.0, np.float32)
    ok = ref * 1.04
    assert og.sgemm_verdict_bad(ok, ref, 8, 8) == 0
    bad = ref.copy()
    bad[2, 3] = 10.6
    bad[2, 5] = 10.6          # same row: counted once
    assert og.sgemm_verdict_bad(bad, ref, 8, 8) == 1
    allbad = ref * 2
    assert og.sgemm_verdict_bad(allbad, ref, 8, 8) == 5


# --------------------------------------------------------------- generators (a17 inputs)
def lcg_python(state, n):
    """gemv_test.c:46-50 restated with Python integers."""
    out = []
    for _ in range(n):
        state = (state * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        out.append(((state >> 40) & 0xFFFFFF) / float(1 << 24))
    return np.array(out, np.float32), state


def test_frand_matches_integer_lcg(sg):
    want, end = lcg_python(42, 1000)
    s = 42
    got = []
    for _ in range(1000):
        v, s = sg.frand(s)
        got.append(v)
    assert np.array_equal(np.array(got, np.float32), want) and s == end


def test_gen_uniform_parallel_equals_serial(sg):
    n = 200_003                          # several 64K chunks, ragged end
    got, end = sg.gen_uniform(n, 7, -0.5)
    want, wend = lcg_python(7, n)
    assert np.array_equal(got, want - np.float32(0.5)) and end == wend


def test_gen_normal_box_muller(sg):
    n = 100_001
    got, end = sg.gen_normal(n, 99, 0.0, 0.02)
    u, wend = lcg_python(99, n + 1)
    assert end == wend
    u1 = np.where(u[0::2] <= 0, 1.0 / (1 << 24), u[0::2].astype(np.float64))
    u2 = u[1::2].astype(np.float64)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * r.size)
    z[0::2] = r * np.cos(2 * math.pi * u2)
    z[1::2] = r * np.sin(2 * math.pi * u2)
    assert np.allclose(got, (0.02 * z[:n]).astype(np.float32), rtol=0, atol=1e-7)
    assert abs(got.mean()) < 3 * 0.02 / math.sqrt(n) * 1.5 and abs(got.std() / 0.02 - 1) < 0.01


def test_f32_to_f16_matches_numpy(sg):
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * 0.02,
        rng.standard_normal(50_000).astype(np.float32) * 1e4,
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 1e-8, 2.0**-25, 2.0**-24, 3 * 2.0**-26,
                  2.0**-14, 2.0**-14 * (1 - 2.0**-11), np.inf, -np.inf], np.float32),
        (np.arange(-3000, 3000, dtype=np.float32) * 2.0**-24).astype(np.float32),
    ])
    got = sg.f32_to_f16(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_srand_fixture(sg):
    """First values of the SGEMM generator (srand(42), interleaved A/B; gpu_workload.c:81-82)."""
    fx = json.load(open(os.path.join(GOLDEN, "sgemm_srand42_head.json")))
    A, B = sg.gen_sgemm_inputs(len(fx["A"]), 42)
    assert np.array_equal(A, np.array(fx["A"], np.float32))
    assert np.array_equal(B, np.array(fx["B"], np.float32))
    # (rand()%2000 - 1000)/1000: a multiple of 0.001 in [-1, 0.999]
    A, B = sg.gen_sgemm_inputs(100_000, 42)
    for v in (A, B):
        assert v.min() >= -1.0 and v.max() <= 0.999
        assert np.allclose(np.round(v * 1000), v * 1000, atol=1e-3)


# -------------------------------------------------- GEMV fp32 (gemv_test.c:85-90, gpt2_engine.c:342-349)
@pytest.mark.parametrize("N,K", [(1, 1), (3, 7), (17, 64), (64, 17), (130, 333)])
def test_gemv_integers_exact(og, N, K):
    rng = np.random.default_rng(N * 7 + K)
    W = rng.integers(-3, 4, (N, K))
    x = rng.integers(-3, 4, K)
    b = rng.integers(-5, 6, N)
    assert np.array_equal(og.gemv(W, x, None, K, N).astype(np.int64), W @ x)
    assert np.array_equal(og.gemv(W, x, b, K, N).astype(np.int64), W @ x + b)
    assert np.array_equal(og.gemv(W, x, b, K, N, nthreads=3), og.gemv(W, x, b, K, N))


def test_gemv_multi_is_rowwise_gemv(og):
    rng = np.random.default_rng(8)
    K, N, T = 96, 40, 19
    W = rng.standard_normal((N, K)).astype(np.float32)
    X = rng.standard_normal((T, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    Y = og.gemv_multi(W, X, b, K, N, T)
    for t in range(T):
        assert np.array_equal(Y[t], og.gemv(W, X[t], b, K, N))
    assert np.array_equal(og.gemv_multi(W, X, None, K, N, 1)[0], og.gemv(W, X[0], None, K, N))


# ------------------------------------------------------ GEMV fp16 (qwen_engine.c:276-284)
def test_gemv_h_integers_exact(og):
    rng = np.random.default_rng(9)
    N, K = 50, 72
    Wi = rng.integers(-8, 9, (N, K))
    Wh = Wi.astype(np.float16).view(np.uint16)
    x = rng.integers(-4, 5, K)
    bi = rng.integers(-9, 10, N)
    bh = bi.astype(np.float16).view(np.uint16)
    assert np.array_equal(og.gemv_h(Wh, x, None, K, N).astype(np.int64), Wi @ x)
    assert np.array_equal(og.gemv_h(Wh, x, bh, K, N).astype(np.int64), Wi @ x + bi)
    assert np.array_equal(og.gemv_h_fbias(Wh, x, bi.astype(np.float32), K, N).astype(np.int64), Wi @ x + bi)


def test_gemv_h_special_codes(og):
    """Subnormal codes contribute 0; exponent-31 codes contribute 2^16 (1 + m/1024)."""
    K = 8
    W = np.array([[0x0001, 0x8001, 0x03ff, 0x8000, 0x7c00, 0xfc01, 0x3c00, 0x0000]], np.uint16)
    x = np.ones(K, np.float32)
    want = 65536.0 - 65536.0 * (1 + 1 / 1024) + 1.0
    assert og.gemv_h(W, x, None, K, 1)[0] == np.float32(want)


# ------------------------------------- GEMV fp16 weights and fp16 x (the fp16-x variant)
def test_gemv_hh_integers_exact(og):
    """Integer fp16 W and x (exact in fp16 and in every fp32 partial sum) against int64,
    with and without bias, N != K (a transposed operand or a dropped bias fails)."""
    rng = np.random.default_rng(19)
    N, K = 37, 200
    Wi = rng.integers(-16, 17, (N, K))
    xi = rng.integers(-16, 17, K)
    bi = rng.integers(-50, 51, N)
    Wh = Wi.astype(np.float16).view(np.uint16)
    xh = xi.astype(np.float16).view(np.uint16)
    assert np.array_equal(og.gemv_hh(Wh, xh, None, K, N).astype(np.int64), Wi @ xi)
    assert np.array_equal(og.gemv_hh(Wh, xh, bi.astype(np.float32), K, N).astype(np.int64), Wi @ xi + bi)


def test_gemv_hh_is_gemv_h_on_ieee_decoded_x(og):
    """On normal x codes (exponent 1..30) the fp16-x GEMV is gemv_h over numpy's IEEE half
    decode of x, bit for bit, at a Qwen shape with the fused-qkv bias."""
    rng = np.random.default_rng(20)
    N, K = 1152, 896
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float16).view(np.uint16)
    x16 = rng.standard_normal(K).astype(np.float16)
    x16[np.abs(x16) < np.float16(2.0 ** -14)] = np.float16(0.5)         # keep every code normal
    bias = (rng.standard_normal(N) * 0.02).astype(np.float32)
    got = og.gemv_hh(W, x16.view(np.uint16), bias, K, N, nthreads=4)
    want = og.gemv_h_fbias(W, x16.astype(np.float32), bias, K, N, nthreads=4)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemv_hh_special_x_codes(og):
    """x codes follow the reference h2f: subnormals and -0 read +0 (IEEE would give nonzero
    subnormals), exponent 31 reads the finite 2^16 (1 + m/1024) (IEEE: inf/NaN)."""
    K = 6
    x = np.array([0x0001, 0x83ff, 0x7c00, 0xfc01, 0x7fff, 0x3c00], np.uint16)
    W = np.eye(K, dtype=np.float16).view(np.uint16)                     # y[n] = decoded x[n]
    y = og.gemv_hh(W, x, None, K, K)
    want = np.array([0.0, 0.0, 65536.0, -65536.0 * (1 + 1 / 1024), 65536.0 * (1 + 1023 / 1024), 1.0], np.float32)
    assert np.array_equal(y, want)
    assert not np.signbit(y[1])


# ---------------------------------------------------------- RMSNorm / RoPE tables
def test_rms_matches_torch(og):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(10)
    x = rng.standard_normal(896).astype(np.float32)
    w = (rng.standard_normal(896) * 0.5).astype(np.float16).view(np.uint16)
    got = og.rms(x, w, 1e-6)
    wf = torch.from_numpy(og.h2f_array(w))
    want = torch.nn.functional.rms_norm(torch.from_numpy(x)[None].double(), (896,), wf.double(), eps=1e-6)[0]
    assert np.allclose(got, want.numpy(), rtol=1e-5, atol=1e-6)


def test_rope_tables_closed_form(og):
    ctx, hd, theta = 300, 64, 1e6
    c, s = og.rope_tables(ctx, hd, theta)
    ang = np.arange(ctx)[:, None] * theta ** (-2.0 * np.arange(hd // 2)[None, :] / hd)
    assert np.array_equal(c, np.cos(ang).astype(np.float32))
    assert np.array_equal(s, np.sin(ang).astype(np.float32))
    assert np.all(c[0] == 1) and np.all(s[0] == 0)


def test_argmax_first_max(og):
    assert og.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
