"""The reference-named GEMV kernels launched the way a host that keeps its own module flow
launches them: the code object read from its file and loaded with hipModuleLoadData, the
kernel resolved by name with hipModuleGetFunction and launched with hipModuleLaunchKernel at
the reference callers' grid (cuModuleLoadData / cuModuleGetFunction / cuLaunchKernel in
gemv_test.c:52-72,108-111, gpt2_engine.c:185,260,280 and qwen_engine.c:219,265), against the
oracle.  Also runs the gemv_test harness, which does the same from C.

Bars as in test_gpu_gemv.py: fp32 weights per element 1e-4 |y_ref| + 1e-4 (gemv_test.c:119);
fp16 weights normwise 1e-3 and per element 1e-3 |y_ref| + 1e-3 max|y_ref|."""
import ctypes as ct
import json
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CO_DIR = os.path.join(ROOT, "switch-l4t-gpu_amd", "build")
BIN = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin")
NT = min(16, os.cpu_count() or 1)
GPT2_SHAPES = [(2304, 768), (768, 768), (3072, 768), (768, 3072), (50257, 768)]      # [N x K]
QWEN_SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896), (1152, 896), (9728, 896)]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Hip:
    """The HIP module API through ctypes, as a C host would call it."""

    def __init__(self):
        self.lib = ct.CDLL("libamdhip64.so")
        self.lib.hipModuleLoadData.argtypes = [ct.POINTER(ct.c_void_p), ct.c_void_p]
        self.lib.hipModuleGetFunction.argtypes = [ct.POINTER(ct.c_void_p), ct.c_void_p, ct.c_char_p]
        self.lib.hipModuleLaunchKernel.argtypes = [ct.c_void_p] + [ct.c_uint] * 7 + [ct.c_void_p,
                                                                                      ct.POINTER(ct.c_void_p),
                                                                                      ct.c_void_p]
        self.lib.hipModuleUnload.argtypes = [ct.c_void_p]
        self.mods = {}

    def module(self, name):
        """The code object build/<name>.co, loaded once (the reference's cuModuleLoadData(PTX))."""
        if name not in self.mods:
            image = open(os.path.join(CO_DIR, name + ".co"), "rb").read()
            buf = ct.create_string_buffer(image, len(image))
            m = ct.c_void_p()
            assert self.lib.hipModuleLoadData(ct.byref(m), buf) == 0, name
            self.mods[name] = (m, buf)
        return self.mods[name][0]

    def function(self, module, sym):
        f = ct.c_void_p()
        assert self.lib.hipModuleGetFunction(ct.byref(f), self.module(module), sym.encode()) == 0, sym
        return f

    def launch(self, f, grid, args):
        """hipModuleLaunchKernel(f, grid, 256 threads, shmem 0, NULL stream, params, NULL)."""
        vals = [ct.c_void_p(a.v) if isinstance(a, Ptr) else (ct.c_void_p(None) if a is None else ct.c_int(a))
                for a in args]
        params = (ct.c_void_p * len(vals))(*[ct.addressof(v) for v in vals])
        gx, gy = grid
        assert self.lib.hipModuleLaunchKernel(f, gx, gy, 1, 256, 1, 1, 0, None, params, None) == 0

    def launch_shape(self, f, grid, block, args):
        """hipModuleLaunchKernel with any block shape; returns HIP's status."""
        vals = [ct.c_void_p(a.v) if isinstance(a, Ptr) else (ct.c_void_p(None) if a is None else ct.c_int(a))
                for a in args]
        params = (ct.c_void_p * len(vals))(*[ct.addressof(v) for v in vals])
        return self.lib.hipModuleLaunchKernel(f, grid, 1, 1, *block, 0, None, params, None)


class Ptr:
    def __init__(self, v):
        self.v = v


@pytest.fixture(scope="module")
def hip(gpu):
    return Hip()


def upload(gpu, a):
    d = gpu.DeviceArray.from_host(np.ascontiguousarray(a))
    return d


def run_gemv(gpu, hip, module, sym, grid, W, x, bias, K, N, T=None):
    dW, dx = upload(gpu, W), upload(gpu, x)
    dy = gpu.DeviceArray(N * (T or 1))
    dy.fill_bytes(0xFF)
    db = upload(gpu, np.asarray(bias, np.float32)) if bias is not None else None
    f = hip.function(module, sym)
    if sym in ("gemv", "gemv4", "gemv_warp"):
        args = [Ptr(dW.ptr), Ptr(dx.ptr), Ptr(dy.ptr), K, N]
    elif sym == "gemv_multi":
        args = [Ptr(dW.ptr), Ptr(dx.ptr), Ptr(db.ptr) if db else None, Ptr(dy.ptr), K, N, T]
    else:
        args = [Ptr(dW.ptr), Ptr(dx.ptr), Ptr(db.ptr) if db else None, Ptr(dy.ptr), K, N]
    hip.launch(f, grid, args)
    gpu.synchronize()
    return dy.to_host()


@pytest.mark.parametrize("N,K", GPT2_SHAPES)
@pytest.mark.parametrize("sym", ["gemv_warp", "gemv_warp_b"])
def test_gpt2_engine_geometry(gpu, hip, og, sym, N, K):
    """gemv_warp / gemv_warp_b from the gpt2_kernels object at (N+7)/8 blocks of 256
    (gpt2_engine.c:185,188,260)."""
    say(f"by name {sym} {N}x{K} grid {(N + 7) // 8}")
    W, s = gpu.gen_normal(N * K, 3 + N, 0.0, 0.02)
    x, s = gpu.gen_normal(K, s, 0.0, 1.0)
    bias = gpu.gen_normal(N, s, 0.0, 0.1)[0] if sym == "gemv_warp_b" else None
    y = run_gemv(gpu, hip, "gpt2_kernels", sym, ((N + 7) // 8, 1), W, x, bias, K, N)
    ref = og.gemv(W, x, bias, K, N, NT)
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref) + 1e-4), np.abs(y - ref).max()


@pytest.mark.parametrize("N,K", QWEN_SHAPES)
@pytest.mark.parametrize("sym", ["gemv_h", "gemv_hh"])
def test_qwen_engine_geometry(gpu, hip, og, sym, N, K):
    """gemv_h (and its fp16-x form gemv_hh) from the qwen_kernels object at (N+7)/8 blocks of
    256 (qwen_engine.c:219,242,249,256,265), the fused qkv shape with its bias."""
    say(f"by name {sym} {N}x{K} grid {(N + 7) // 8}")
    Wf, s = gpu.gen_normal(N * K, 5 + N, 0.0, 0.02)
    W = gpu.f32_to_f16(Wf)
    xf, s = gpu.gen_normal(K, s, 0.0, 1.0)
    bias = gpu.gen_normal(N, s, 0.0, 0.02)[0] if N == 1152 else None
    if sym == "gemv_h":
        y = run_gemv(gpu, hip, "qwen_kernels", sym, ((N + 7) // 8, 1), W, xf, bias, K, N)
        ref = og.gemv_h_fbias(W, xf, bias, K, N, NT)
    else:
        x16 = gpu.f32_to_f16(xf)
        y = run_gemv(gpu, hip, "qwen_kernels", sym, ((N + 7) // 8, 1), W, x16, bias, K, N)
        ref = og.gemv_hh(W, x16, bias, K, N, NT)
    m = np.abs(ref).max()
    assert np.abs(y - ref).max() / m <= 1e-3
    assert np.all(np.abs(y - ref) <= 1e-3 * np.abs(ref) + 1e-3 * m)


@pytest.mark.parametrize("T", [1, 8, 17, 128])
@pytest.mark.parametrize("N,K", [(2304, 768), (768, 3072)])
def test_gemv_multi_prefill_geometry(gpu, hip, og, N, K, T):
    """gemv_multi from the gpt2_kernels object at ((N+7)/8, (T+15)/16) blocks of 256
    (gpt2_engine.c:280), with the qkv bias."""
    say(f"by name gemv_multi {N}x{K} T={T}")
    W, s = gpu.gen_normal(N * K, 9 + T, 0.0, 0.02)
    X, s = gpu.gen_normal(T * K, s, 0.0, 1.0)
    bias, _ = gpu.gen_normal(N, s, 0.0, 0.1)
    Y = run_gemv(gpu, hip, "gpt2_kernels", "gemv_multi", ((N + 7) // 8, (T + 15) // 16), W, X, bias, K, N, T=T)
    ref = og.gemv_multi(W, X, bias, K, N, T, NT).reshape(-1)
    assert np.all(np.abs(Y - ref) <= 1e-4 * np.abs(ref) + 1e-4), np.abs(Y - ref).max()


@pytest.mark.parametrize("sym,grid", [("gemv", lambda N: (N + 255) // 256), ("gemv4", lambda N: (N + 255) // 256),
                                      ("gemv_warp", lambda N: (N + 7) // 8)])
def test_gemv_test_geometry(gpu, hip, og, sym, grid):
    """gemv / gemv4 / gemv_warp from the gemv object at gemv_test.c:108's geometry, on its
    default 4096 x 4096 problem with frand() - 0.5 inputs (gemv_test.c:80-81)."""
    N = K = 4096
    say(f"by name {sym} {N}x{K} grid {grid(N)}")
    W, s = gpu.gen_uniform(N * K, 42, -0.5)
    x, _ = gpu.gen_uniform(K, s, -0.5)
    y = run_gemv(gpu, hip, "gemv", sym, (grid(N), 1), W, x, None, K, N)
    ref = og.gemv(W, x, None, K, N, NT)
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref) + 1e-4), np.abs(y - ref).max()


# K values that put the by-name symbols on each of their three team shapes (16-, 64- and
# 256-lane teams) and past them on the wave-per-row kernel, for 4 fp32 / 8 fp16 per segment.
BYNAME_INT = [(1000, 64), (37, 512), (300, 1024), (129, 2048), (65, 4096), (33, 8192), (5, 9000), (3, 20000)]


@pytest.mark.parametrize("N,K", BYNAME_INT)
@pytest.mark.parametrize("module,sym", [("gemv", "gemv"), ("gpt2_kernels", "gemv_warp_b"), ("qwen_kernels", "gemv_h"),
                                        ("qwen_kernels", "gemv_hh")])
def test_integer_exact_reference_geometry(gpu, hip, module, sym, N, K):
    """Integer-valued operands at the reference geometry ((N+255)/256 blocks for gemv, (N+7)/8
    otherwise), K reaching every team shape and the wave-per-row kernel: exact results."""
    say(f"by name {sym} integer {N}x{K}")
    rng = np.random.default_rng(N + 7 * K)
    Wi, xi, bi = rng.integers(-3, 4, (N, K)), rng.integers(-3, 4, K), rng.integers(-5, 6, N)
    half = sym in ("gemv_h", "gemv_hh")
    W = Wi.astype(np.float16).view(np.uint16) if half else Wi.astype(np.float32)
    x = xi.astype(np.float16).view(np.uint16) if sym == "gemv_hh" else xi.astype(np.float32)
    bias = bi.astype(np.float32) if sym != "gemv" else None
    grid = (N + 255) // 256 if sym == "gemv" else (N + 7) // 8
    y = run_gemv(gpu, hip, module, sym, (grid, 1), W, x, bias, K, N)
    assert np.array_equal(y, (Wi @ xi + (bi if bias is not None else 0)).astype(np.float32))


@pytest.mark.parametrize("N,K", [(41, 896), (37, 4864)])
@pytest.mark.parametrize("sym", ["gemv_h", "gemv_hh"])
def test_special_codes_reference_geometry(gpu, hip, og, sym, N, K):
    """The fp16 by-name symbols at (N+7)/8 blocks, narrow (16-lane teams) and wide (64-lane
    teams, two rows each; N odd leaves the last team one row) rows, x staged in LDS: subnormal
    and -0 codes read +0, exponent-31 codes 2^16 (1 + m/1024) in W and, for gemv_hh, in x
    (rows whose fast sum is not finite are recomputed with the exact decode).  Integer-valued
    operands keep every partial sum exact, so the results are compared bit for bit with the
    oracle's serial decode."""
    say(f"by name {sym} special codes {N}x{K}")
    rng = np.random.default_rng(N * K)
    big = np.concatenate([np.arange(0x7c00, 0x8000), np.arange(0xfc00, 0x10000)]).astype(np.uint16)
    small = np.concatenate([np.arange(0, 1024), np.arange(0x8000, 0x8400),
                            np.array([0x3c00, 0x4000, 0x4200, 0xbc00, 0xc000] * 60)]).astype(np.uint16)
    W = rng.choice(small, (N, K)).astype(np.uint16)
    xbig = rng.choice(K, 4, replace=False)         # exponent-31 x positions (gemv_hh)
    cols = np.setdiff1d(np.arange(K), xbig)        # exponent-31 weights elsewhere: no big x big product
    for r in range(0, N, 3):                       # exponent-31 weights in every third row
        W[r, rng.choice(cols, 8, replace=False)] = rng.choice(big, 8)
    xi = rng.integers(-2, 3, K)
    bias = rng.integers(-5, 6, N).astype(np.float32)
    grid = ((N + 7) // 8, 1)
    if sym == "gemv_h":
        x = xi.astype(np.float32)
        y = run_gemv(gpu, hip, "qwen_kernels", sym, grid, W, x, bias, K, N)
        ref = og.gemv_h_fbias(W, x, bias, K, N, NT)
    else:
        x16 = xi.astype(np.float16).view(np.uint16)
        x16[rng.choice(cols, 16, replace=False)] = rng.choice(small[:2048], 16)   # subnormal, -0
        x16[xbig] = rng.choice(big, 4)                                            # exponent 31
        y = run_gemv(gpu, hip, "qwen_kernels", sym, grid, W, x16, bias, K, N)
        ref = og.gemv_hh(W, x16, bias, K, N, NT)
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("co,args", [("gemv", ["4096", "4096"]), ("gpt2_kernels", ["2304", "768", "--bias"]),
                                     ("qwen_kernels", ["151936", "896", "--h", "--normal"]),
                                     ("qwen_kernels", ["9728", "896", "--hh", "--normal"]),
                                     ("gpt2_kernels", ["2304", "768", "--multi", "128"])])
def test_gemv_test_harness(gpu, co, args):
    """The C harness end to end: module by path, kernels by name, reference geometry, its own
    serial golden; every kernel CORRECT and the done flag set."""
    cmd = [os.path.join(BIN, "gemv_test"), os.path.join(CO_DIR, co + ".co")] + args + ["--json"]
    say("run", " ".join(cmd))
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    d = json.loads(out.stdout)
    assert d["done"] is True and d["kernels"]
    assert all(k["verdict"] == "CORRECT" and k["gbps"] > 0 for k in d["kernels"])
    if co == "gemv":
        assert [k["kernel"] for k in d["kernels"]] == ["gemv", "gemv4", "gemv_warp"]


# The K-over-waves SGEMM members by name at grids smaller than their tile count: each block
# strides over several tiles (the staging reused tile after tile; with sgemm_kwave_edge, the
# clamped edge tiles and, N % 64 == 1, the tiles that also compute column N-1).
BYNAME_KWAVE = [("sgemm_kwave", 256, 320, 544, 5), ("sgemm_kwave", 128, 192, 1024, 1),
                ("sgemm_kwave_edge", 1023, 1025, 997, 7), ("sgemm_kwave_edge", 200, 191, 33, 3),
                ("sgemm_kwave_edge", 130, 65, 40, 1), ("sgemm_kwave_edge", 1000, 1000, 1000, 64),
                ("sgemm_kwave128", 384, 512, 544, 5), ("sgemm_kwave128", 256, 256, 1024, 1),
                ("sgemm_kwave128", 2048, 2048, 256, 100)]


@pytest.mark.parametrize("sym,M,N,K,grid", BYNAME_KWAVE)
def test_kwave_members_by_name_any_grid(gpu, hip, sym, M, N, K, grid):
    say(f"by name {sym} {M}x{N}x{K} grid {grid}")
    rng = np.random.default_rng(M + 3 * N + 7 * K + grid)
    A = rng.integers(-2, 3, (M, K)).astype(np.float32)
    B = rng.integers(-2, 3, (K, N)).astype(np.float32)
    want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    dA, dB, dC = upload(gpu, A), upload(gpu, B), gpu.DeviceArray((M, N))
    dC.fill_bytes(0xFF)
    hip.launch(hip.function("switch_gpu", sym), (grid, 1), [Ptr(dA.ptr), Ptr(dB.ptr), Ptr(dC.ptr), M, N, K])
    gpu.synchronize()
    assert np.array_equal(dC.to_host(), want)


def test_block_beyond_launch_bound_refused(gpu, hip):
    """The kernels' block-size checks (sgpu_block256) read no z size: a block of x*y == 256
    threads has z == 1 because HIP refuses a launch whose block holds more threads than the
    kernel's __launch_bounds__(256).  This pins that refusal, for a by-name GEMV symbol and an
    SGEMM member: the launch returns an error and nothing is written."""
    N, K = 1024, 896
    dW, dx, dy = gpu.DeviceArray(N * K // 2), gpu.DeviceArray(K), gpu.DeviceArray(N)
    dy.fill_bytes(0xFF)
    f = hip.function("qwen_kernels", "gemv_h")
    say("gemv_h launched with a 256x1x2 block")
    assert hip.launch_shape(f, N // 8, (256, 1, 2), [Ptr(dW.ptr), Ptr(dx.ptr), None, Ptr(dy.ptr), K, N]) != 0
    n = 256
    dA, dB, dC = gpu.DeviceArray((n, n)), gpu.DeviceArray((n, n)), gpu.DeviceArray((n, n))
    dC.fill_bytes(0xFF)
    g = hip.function("switch_gpu", "sgemm_tiled")
    say("sgemm_tiled launched with a 128x2x2 block")
    assert hip.launch_shape(g, 16, (128, 2, 2), [Ptr(dA.ptr), Ptr(dB.ptr), Ptr(dC.ptr), n, n, n]) != 0
    gpu.synchronize()
    assert np.all(np.isnan(dy.to_host())) and np.all(np.isnan(dC.to_host()))


@pytest.mark.parametrize("block", [(64, 2, 2), (32, 2, 4), (128, 1, 2)])
def test_three_d_blocks(gpu, hip, og, block):
    """gemv_h launched by name with 3-D blocks of 256 threads (the wave-per-row path): every
    row against the oracle.  Each z layer of a block has its own thread indices."""
    N, K = 1000, 896
    say(f"by name gemv_h {N}x{K} block {block}")
    Wf, s = gpu.gen_normal(N * K, 11, 0.0, 0.02)
    W = gpu.f32_to_f16(Wf)
    x, s = gpu.gen_normal(K, s, 0.0, 1.0)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    dW, dx, db = upload(gpu, W), upload(gpu, x), upload(gpu, bias)
    dy = gpu.DeviceArray(N)
    dy.fill_bytes(0xFF)
    f = hip.function("qwen_kernels", "gemv_h")
    assert hip.launch_shape(f, (N + 3) // 4, block, [Ptr(dW.ptr), Ptr(dx.ptr), Ptr(db.ptr), Ptr(dy.ptr), K, N]) == 0
    gpu.synchronize()
    y = dy.to_host()
    ref = og.gemv_h_fbias(W, x, bias, K, N, NT)
    m = np.abs(ref).max()
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref) + 1e-4 * m), np.abs(y - ref).max()
