"""Benchmark of the matmul hot path on one MI355X; prints ONE JSON line.

Metric (headline): SGEMM TFLOPS at 4096^3 fp32 + batch-1 GEMV GB/s (fraction of HBM peak)
+ decode tok/s.  `value` is the SGEMM figure: a step is one C = A*B, M = N = K = 4096, fp32
row-major, A and B from the reference generator (srand(42), gpu_workload.c:81-82), computed
by sgpu_sgemm_opt through libswitchgpu.so (the member its plan picks at this shape, named
in the line's config: the K-over-waves member sgemm_kwave).  One verified launch, then W untimed warm-up steps immediately followed by exactly K
timed steps between device synchronisations.  Inputs are resident in HBM before timing starts.

Secondary figures measured in the same run (same JSON line):
  gemv   -- fp16-weight GEMV on the Qwen2.5-0.5B lm_head shape [151936 x 896], rotating
            four weight copies (1.09 GB) so every launch streams from HBM, not the MALL
  sgemm_sweep -- sgpu_sgemm_opt at 256^3 .. 4096^3 and the ragged 1023x1025x997
  gemv_shapes -- every GPT-2 (fp32) and Qwen2.5-0.5B (fp16) projection shape
  Both report the time per launch replayed from a recorded graph (rates are computed from it)
  and per launch from a host loop of ctypes calls (which adds the host's submission cost).
  decode -- random-init Qwen2.5-0.5B-architecture decode, 32-token prompt, 128 greedy tokens
  gemv_hh -- the same lm_head with fp16 x (sgpu_gemv_hh), its own HBM roofline
Clocks: before the counted warm-up, SGEMM launches run for a stated settling time (the GPU
clock climbs from idle over tens of milliseconds); the steady-state kernel time of a longer
event-timed loop after the timed steps is reported beside `value`.
CPU baselines (the oracle, i.e. the restated reference CPU goldens, on the host's cores --
the threads used, the CPU model and the visible core count are in each entry): the SGEMM on a
bounded sample of rows of the same 4096^3 problem (top-level cpu_baseline); og_gemv_h on the
lm_head shape (gemv.cpu_baseline); og_qwen_forward on the same random-init model for a few
positions (decode.cpu_baseline); each row-parallel over the threads and, for the GEMV and
decode, also on one thread in the reference's serial form.
"""
import argparse
import ctypes as ct
import itertools
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "switch-l4t-gpu_amd"))

import numpy as np  # noqa: E402

import sgpu  # noqa: E402

METRIC = "SGEMM TFLOPS @4096³ + GEMV GB/s (% of HBM peak); decode tok/s"
PEAK_FP32_MATRIX_TFLOPS = 157.3      # MI355X dense fp32 matrix
PEAK_HBM_GBPS = 8000.0               # MI355X HBM3E
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_info():
    """CPU model and core counts of the host running the bench."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "cpu_count": os.cpu_count(), "cpus_available": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_threads():
    """Threads for the row-parallel CPU legs: every core this process may use, capped by
    OMP_NUM_THREADS when it is set (the host's CPU share for one GPU)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def bench_sgemm(n, steps, warmup, settle_s=0.3, steady_launches=200):
    A, B = sgpu.gen_sgemm_inputs(n * n, 42)
    dA, dB, dC = sgpu.DeviceArray.from_host(A), sgpu.DeviceArray.from_host(B), sgpu.DeviceArray((n, n))
    run = lambda: sgpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, n, n, n, None)
    run()
    sgpu.synchronize()
    # correctness of what is timed: sampled rows against the oracle-free float64 product
    C = dC.to_host()
    rows = np.linspace(0, n - 1, 8).astype(int)
    ref = A.reshape(n, n)[rows].astype(np.float64) @ B.reshape(n, n).astype(np.float64)
    err = float(np.abs(C[rows] - ref).max() / np.abs(ref).max())
    # clock settling, then the counted warm-up right before the timed launches: the GPU clock
    # climbs from idle over tens of milliseconds, and a host-side pause between warm-up and
    # timing would let it fall again
    settle = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < settle_s:
        for _ in range(20):
            run()
        sgpu.synchronize()
        settle += 20
    ev = sgpu.Events()
    for _ in range(warmup):
        run()
    sgpu.synchronize()
    t0 = time.perf_counter()
    ev.record_start(None)
    for _ in range(steps):
        run()
    ev.record_stop(None)
    sgpu.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = ev.elapsed_ms() / steps
    # steady state beside it: a longer event-timed loop straight after the timed steps
    ev.record_start(None)
    for _ in range(steady_launches):
        run()
    ev.record_stop(None)
    sgpu.synchronize()
    steady_ms = ev.elapsed_ms() / steady_launches
    flops = 2.0 * n * n * n
    return dict(wall_s=wall, kernel_ms=kernel_ms, flops=flops, err=err, settle_launches=settle, settle_s=settle_s,
                steady_ms=steady_ms, steady_launches=steady_launches)


def flush_subnormal_f16(codes):
    """float64 values of fp16 codes with the h2f contract's flush of subnormals to 0."""
    v = np.asarray(codes, np.uint16).view(np.float16).astype(np.float64)
    v[np.abs(v) < 2.0 ** -14] = 0.0
    return v


def bench_gemv_lm_head(reps=100, copies=4, warm=1000, x16=False):
    """The lm_head GEMV [151936 x 896], fp16 weights: sgpu_gemv_h (fp32 x) or, with x16,
    sgpu_gemv_hh (fp16 x)."""
    N, K = 151936, 896
    Wf, s = sgpu.gen_normal(N * K, 42, 0.0, 0.02)
    W = sgpu.f32_to_f16(Wf)
    del Wf
    x, _ = sgpu.gen_normal(K, s, 0.0, 1.0)
    xin = sgpu.f32_to_f16(x) if x16 else x
    dWs = [sgpu.DeviceArray.from_host(W) for _ in range(copies)]
    dx, dy = sgpu.DeviceArray.from_host(xin), sgpu.DeviceArray(N)
    fn = "sgpu_gemv_hh" if x16 else "sgpu_gemv_h"
    run = lambda i: sgpu.call(fn, dWs[i % copies].ptr, dx.ptr, None, dy.ptr, K, N, None)
    for i in range(copies * 2):
        run(i)
    sgpu.synchronize()
    y = dy.to_host()
    rows = np.arange(0, N, 997)
    Wd = flush_subnormal_f16(W.reshape(N, K)[rows])        # the h2f contract flushes fp16 subnormals
    ref = Wd @ (flush_subnormal_f16(xin) if x16 else x.astype(np.float64))
    err = float(np.abs(y[rows] - ref).max() / np.abs(ref).max())
    ev = sgpu.Events()
    for i in range(warm):                      # ~45 ms: clocks to steady state, then timed
        run(i)
    sgpu.synchronize()
    ev.record_start(None)
    for i in range(reps * copies):
        run(i)
    ev.record_stop(None)
    us = ev.elapsed_ms() * 1e3 / (reps * copies)
    algo_bytes = 2.0 * N * K + (2.0 if x16 else 4.0) * K + 4.0 * N
    for d in dWs + [dx, dy]:
        d.close()
    return dict(us=us, bytes=algo_bytes, gbps=algo_bytes / (us * 1e-6) / 1e9, err=err, copies=copies, W=W, x=x)


# In order of size.  A shape timed right after 4096^3 (about 0.6 s of the chip at full matrix
# load) runs slower than the same shape timed before it: 1023x1025x997 took 20.7-21.3 us a launch
# in a graph straight after 4096^3, 20.5 after a 0.5 s pause, and 20.2 before any large shape.
SWEEP_SHAPES = [(256, 256, 256), (512, 512, 512), (1023, 1025, 997), (1024, 1024, 1024), (2048, 2048, 2048),
                (4096, 4096, 4096)]
GEMV_SHAPES = [("fp32", "gpt2 qkv", 2304, 768), ("fp32", "gpt2 attn-out", 768, 768), ("fp32", "gpt2 fc", 3072, 768),
               ("fp32", "gpt2 proj", 768, 3072), ("fp32", "gpt2 lm_head", 50257, 768),
               ("fp16", "qwen q", 896, 896), ("fp16", "qwen k/v", 128, 896), ("fp16", "qwen o", 896, 896),
               ("fp16", "qwen gate/up", 4864, 896), ("fp16", "qwen down", 896, 4864),
               ("fp16", "qwen lm_head", 151936, 896), ("fp16", "qwen qkv fused +bias", 1152, 896),
               ("fp16", "qwen gate|up fused", 9728, 896)]
GEMV_SHAPES += [("fp16x", name, N, K) for wt, name, N, K in GEMV_SHAPES if wt == "fp16"]
ROTATE_BYTES = 600e6     # weight copies rotated per shape, up to 64: past the 256 MB MALL where that fits


def warm_for(launch, sync, min_launches, min_s):
    """Run `launch` at least min_launches times and for at least min_s seconds of wall time,
    synchronising every 10 launches: the clock climbs from idle over tens of milliseconds,
    and a count-only warm-up of small launches ends before it has (2048^3 timed 142 us per
    launch from a host loop after 50 launches, 128 us after a further second of work)."""
    n, t0 = 0, time.perf_counter()
    while n < min_launches or time.perf_counter() - t0 < min_s:
        for _ in range(10):
            launch()
        n += 10
        sync()
    return n


def bench_sgemm_sweep(reps=100, warm=50, graphs=True, warm_s=0.1, cpu=False):
    """sgpu_sgemm_opt over the SGEMM size sweep (square 256..4096 and the ragged 1023x1025x997),
    reference-generator inputs; HIP-event time per launch after a warm-up of at least `warm`
    launches and `warm_s` seconds, normwise error of sampled rows against a float64 product.
    graphs=False skips the recorded-graph timing (a kernel trace of graph replay is not taken
    by the profiler).  cpu=True adds, at the reference's own sizes (up to 1024, and the ragged
    shape), the oracle's serial SGEMM on one thread -- the reference CPU golden's form
    (gpu_workload.c:97-98) -- timed on the same inputs."""
    out = []
    cus = sgpu.device_props().compute_units
    for M, N, K in SWEEP_SHAPES:
        S = ct.c_int()
        launch = f"{sgpu.lib().sgpu_sgemm_opt_plan(M, N, K, cus, ct.byref(S)).decode()} S={S.value}"
        A, B = sgpu.gen_sgemm_inputs(max(M * K, K * N), 42)
        A, B = A[:M * K], B[:K * N]
        dA, dB, dC = sgpu.DeviceArray.from_host(A), sgpu.DeviceArray.from_host(B), sgpu.DeviceArray((M, N))
        run = lambda: sgpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, M, N, K, None)
        run()
        sgpu.synchronize()
        C = dC.to_host()
        rows = np.linspace(0, M - 1, 8).astype(int)
        ref = A.reshape(M, K)[rows].astype(np.float64) @ B.reshape(K, N).astype(np.float64)
        err = float(np.abs(C[rows] - ref).max() / np.abs(ref).max())
        cpu_row = {}
        if cpu and max(M, N, K) <= 1025:
            t = time.perf_counter()
            _oracle().sgemm_rows(A, B, M, N, K, 0, M, 1)
            dt = time.perf_counter() - t
            cpu_row = {"cpu_1thread_ms": round(dt * 1e3, 1), "cpu_1thread_gflops": round(2.0 * M * N * K / dt / 1e9, 3)}
        ev = sgpu.Events()
        warm_for(run, sgpu.synchronize, warm, warm_s)
        for _ in range(10):
            run()
        ev.record_start(None)
        for _ in range(reps):
            run()
        ev.record_stop(None)
        us = ev.elapsed_ms() * 1e3 / reps
        if not graphs:
            out.append({"M": M, "N": N, "K": K, "launch": launch, "us_host_loop": round(us, 2), "normwise_err": err,
                        **cpu_row})
            for d in (dA, dB, dC):
                d.close()
            continue
        # the same launches recorded once and replayed: no host submission cost per launch.
        # One launch on the stream before recording gives it its split-K workspace (a stream
        # being recorded cannot get one, and sgpu_sgemm_opt would record its unsplit member).
        st = sgpu.Stream()
        sgpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, M, N, K, st.h)
        st.synchronize()
        # 50 launches a graph (the graph launch's own cost spread thin), the median of five
        # event-timed replays
        per_graph, replays = 50, 5
        with sgpu.Graph(st) as g:
            for _ in range(per_graph):
                sgpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, M, N, K, st.h)
        warm_for(g.launch, st.synchronize, max(1, warm // per_graph), warm_s)
        g.launch()
        times = []
        for _ in range(replays):
            ev.record_start(st.h)
            g.launch()
            ev.record_stop(st.h)
            times.append(ev.elapsed_ms() * 1e3 / per_graph)
        us_g = float(np.median(times))
        g.close()
        st.close()
        tf = 2.0 * M * N * K / (us_g * 1e-6) / 1e12
        # the reference's own timing form (events around a host loop of launches,
        # gpu_workload.c:133-139) beside the graph replay's
        tf_loop = 2.0 * M * N * K / (us * 1e-6) / 1e12
        out.append({"M": M, "N": N, "K": K, "launch": launch, "us_in_graph": round(us_g, 2), "us_host_loop": round(us, 2),
                    "tflops": round(tf, 2), "frac": round(tf / PEAK_FP32_MATRIX_TFLOPS, 4),
                    "frac_host_loop": round(tf_loop / PEAK_FP32_MATRIX_TFLOPS, 4), "normwise_err": err,
                    **cpu_row})
        for d in (dA, dB, dC):
            d.close()
    return out


def bench_gemv_shapes(reps=50, warm=100, cpu=False):
    """The per-projection GEMV shapes of both decoders: GPT-2 fp32 through sgpu_gemv_warp_b
    (zero bias, the engine's call), Qwen fp16 through sgpu_gemv_h (fp32 x; the fused qkv shape
    with its bias) and through sgpu_gemv_hh (fp16 x, rows "fp16x").  Weights N(0, 0.02),
    x N(0, 1); copies of W are rotated so consecutive launches read different memory.
    cpu=True adds the oracle's serial GEMV of the same W and x on one thread (the reference
    CPU goldens' form, gemv_test.c:85-90 and qwen_engine.c:276-284), best of 3."""
    out = []
    st = 7
    for wt, name, N, K in GEMV_SHAPES:
        Wf, st = sgpu.gen_normal(N * K, st, 0.0, 0.02)
        x, st = sgpu.gen_normal(K, st, 0.0, 1.0)
        half = wt in ("fp16", "fp16x")
        W = sgpu.f32_to_f16(Wf) if half else Wf
        del Wf
        xin = sgpu.f32_to_f16(x) if wt == "fp16x" else x
        with_bias = "+bias" in name
        bias = sgpu.gen_normal(N, st, 0.0, 0.02)[0] if with_bias else None
        wbytes = W.nbytes
        copies = int(max(2, min(64, np.ceil(ROTATE_BYTES / wbytes))))
        dWs = [sgpu.DeviceArray.from_host(W) for _ in range(copies)]
        dx, dy = sgpu.DeviceArray.from_host(xin), sgpu.DeviceArray(N)
        dz = sgpu.DeviceArray.from_host(np.zeros(N, np.float32) if bias is None else bias) \
            if (wt == "fp32" or with_bias) else None
        if wt == "fp32":
            run = lambda i, st=None: sgpu.call("sgpu_gemv_warp_b", dWs[i % copies].ptr, dx.ptr, dz.ptr, dy.ptr,
                                               K, N, st)
        else:
            fn = "sgpu_gemv_hh" if wt == "fp16x" else "sgpu_gemv_h"
            run = lambda i, st=None, fn=fn: sgpu.call(fn, dWs[i % copies].ptr, dx.ptr, dz.ptr if dz else None,
                                                      dy.ptr, K, N, st)
        run(0)
        sgpu.synchronize()
        y = dy.to_host()
        rows = np.arange(0, N, max(1, N // 64))
        Wd = flush_subnormal_f16(W.reshape(N, K)[rows]) if half else W.reshape(N, K)[rows].astype(np.float64)
        ref = Wd @ (flush_subnormal_f16(xin) if wt == "fp16x" else x.astype(np.float64))
        if bias is not None:
            ref = ref + bias[rows].astype(np.float64)
        err = float(np.abs(y[rows] - ref).max() / np.abs(ref).max())
        ev = sgpu.Events()
        launches = itertools.count()
        warm_for(lambda: run(next(launches)), sgpu.synchronize, warm, 0.05)
        ev.record_start(None)
        for i in range(reps * copies):
            run(i)
        ev.record_stop(None)
        us = ev.elapsed_ms() * 1e3 / (reps * copies)
        # in-graph: one launch per weight copy recorded once, the graph replayed
        strm = sgpu.Stream()
        with sgpu.Graph(strm) as g:
            for i in range(copies):
                run(i, strm.h)
        warm_for(g.launch, strm.synchronize, max(1, warm // copies), 0.05)
        ev.record_start(strm.h)
        for _ in range(reps):
            g.launch()
        ev.record_stop(strm.h)
        us_g = ev.elapsed_ms() * 1e3 / (reps * copies)
        g.close()
        strm.close()
        algo = wbytes + (2.0 if wt == "fp16x" else 4.0) * K + 4.0 * N + (4.0 * N if dz is not None else 0.0)
        gbps = algo / (us_g * 1e-6) / 1e9
        cpu_row = {}
        if cpu:
            og = _oracle()
            if wt == "fp32":
                fcpu = lambda: og.gemv(W, x, np.zeros(N, np.float32), K, N, 1)
            elif wt == "fp16x":
                fcpu = lambda: og.gemv_hh(W, xin, bias, K, N, 1)
            else:
                fcpu = lambda: og.gemv_h_fbias(W, x, bias, K, N, 1)
            best = 1e9
            for _ in range(3):
                t = time.perf_counter()
                fcpu()
                best = min(best, time.perf_counter() - t)
            cpu_row = {"cpu_1thread_us": round(best * 1e6, 1), "cpu_1thread_gbps": round(algo / best / 1e9, 3)}
        out.append({"shape": [N, K], "name": name, "weights": "fp16" if half else "fp32",
                    "x": "fp16" if wt == "fp16x" else "fp32", "us_in_graph": round(us_g, 3),
                    "us_host_loop": round(us, 3), "gbps": round(gbps, 1), "frac_hbm": round(gbps / PEAK_HBM_GBPS, 4),
                    "rotated_mb": round(copies * wbytes / 1e6, 1), "normwise_err": err, **cpu_row})
        for d in dWs + [dx, dy] + ([dz] if dz is not None else []):
            d.close()
        del dWs
    return out


def host_loop_tok_s(eng, ids, gen):
    """The reference's generation loop shape: logits to the host and argmax there per token."""
    for p, tok in enumerate(ids):
        logits = eng.forward(tok, p, p == len(ids) - 1)
    nxt = int(np.argmax(logits))
    t0 = time.perf_counter()
    for g in range(gen):
        logits = eng.forward(nxt, len(ids) + g, True)
        nxt = int(np.argmax(logits))
    return gen / (time.perf_counter() - t0)


def bench_decode(prompt_len=32, gen=128, path=sgpu.QWEN_PATH_GRAPH, compare=True, keep_blob=False):
    cfg = sgpu.qwen_default_cfg()
    t = time.perf_counter()
    blob = sgpu.qwen_random_blob(cfg, seed=2024, std=0.02)
    eng = sgpu.QwenEngine(cfg, blob, path)
    if not keep_blob:
        del blob
        blob = None
    log(f"decode: weights built and uploaded in {time.perf_counter() - t:.1f} s")
    ids = [int(v) for v in np.random.default_rng(32).integers(0, cfg.V, prompt_len)]
    eng.generate(ids, 4)                      # captures the graphs
    sgpu.synchronize()
    # greedy decode timed as (prompt + gen positions) minus (prompt only): prefill excluded
    t0 = time.perf_counter()
    toks = eng.generate(ids, gen)
    t_full = time.perf_counter() - t0
    t0 = time.perf_counter()
    eng.generate(ids, 0)
    t_prefill = time.perf_counter() - t0
    dt = t_full - t_prefill
    host_graph = host_loop_tok_s(eng, ids, gen) if compare else 0.0
    eng.set_path(sgpu.QWEN_PATH_REFERENCE)
    host_ref = host_loop_tok_s(eng, ids, 32) if compare else 0.0
    eng.close()
    log(f"decode: first ids {toks[:8].tolist()}; host-loop tok/s graph {host_graph:.1f}, "
        f"reference launch sequence {host_ref:.1f}")
    per_layer = (cfg.C + (cfg.C + 2 * cfg.NKV * cfg.HD) * cfg.C + cfg.C * cfg.C + cfg.C
                 + 2 * cfg.FC * cfg.C + cfg.C * cfg.FC) * 2 + (cfg.C + 2 * cfg.NKV * cfg.HD) * 4
    bytes_tok = per_layer * cfg.NL + 2 * cfg.V * cfg.C + 2 * cfg.C
    tps = gen / dt
    return dict(tok_s=tps, ms_per_tok=dt / gen * 1e3, bytes_per_token=bytes_tok,
                hbm_floor_frac=bytes_tok * tps / (PEAK_HBM_GBPS * 1e9), prompt=prompt_len, generated=gen,
                prefill_ms=t_prefill * 1e3, host_loop_graph=host_graph, host_loop_reference=host_ref,
                cfg=cfg, blob=blob, ids=ids)


def bench_gpt2_decode(prompt_len=8, gen=128):
    """GPT-2 124M (random-init fp32 weights), graph path with the greedy loop on the device:
    decode tok/s over `gen` positions after the reference's deterministic 8-id prompt."""
    cfg = sgpu.gpt2_cfg()
    w = sgpu.gpt2_random_weights(cfg, 42, 0.03)
    eng = sgpu.Gpt2Engine(cfg, w, sgpu.GPT2_PATH_GRAPH)
    del w
    ids = [(i * 7919 + 42) % cfg.V for i in range(prompt_len)]
    eng.generate(ids, 4)                          # captures the graphs
    sgpu.synchronize()
    t0 = time.perf_counter()
    eng.generate(ids, gen)
    t_full = time.perf_counter() - t0
    t0 = time.perf_counter()
    eng.generate(ids, 0)
    t_prefill = time.perf_counter() - t0
    eng.close()
    dt = t_full - t_prefill
    bytes_tok = 4 * sgpu.lib().sgpu_gpt2_file_floats(ct.byref(cfg)) - 4 * cfg.CTX * cfg.C   # all weights but wpe
    tps = gen / dt
    return dict(tok_s=tps, ms_per_tok=dt / gen * 1e3, bytes_per_token=bytes_tok,
                hbm_floor_frac=bytes_tok * tps / (PEAK_HBM_GBPS * 1e9), prompt=prompt_len, generated=gen,
                prefill_ms=t_prefill * 1e3)


def decode_floor(quick=False):
    """The decode structure's cost model, measured: bin/decode_floor's dependent-launch,
    per-phase weight-streaming floor and AQL dispatch legs, and the engine's own in-graph time
    per launch of each decode phase (sgpu_qwen_phase_times) at three cache lengths, on the
    random-init Qwen2.5-0.5B-architecture model."""
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "decode_floor")
    log(f"decode floor: {exe}")
    r = subprocess.run([exe] + (["--quick"] if quick else []), capture_output=True, text=True, timeout=600)
    sys.stderr.write(r.stderr)
    if r.returncode != 0:
        raise SystemExit(f"decode_floor exited {r.returncode}")
    floor = json.loads(r.stdout)
    cfg = sgpu.qwen_default_cfg()
    eng = sgpu.QwenEngine(cfg, sgpu.qwen_random_blob(cfg, seed=2024, std=0.02), sgpu.QWEN_PATH_FUSED)
    phases = {}
    for pos in (32, 96, 160):
        ph = eng.phase_times(pos, reps=10 if quick else 30)
        layer = sum(ph[k] for k in ("qkv", "attention", "o", "gate_up", "down"))
        ph["layer"] = layer
        ph["token_sum"] = layer * cfg.NL + ph["lm_head"] + ph["argmax_embed"]
        phases[str(pos)] = {k: round(v, 3) for k, v in ph.items()}
        log(f"decode phases at position {pos}: " + ", ".join(f"{k} {v:.2f}" for k, v in ph.items()) + " us")
    eng.close()
    return {"decode_floor": floor, "decode_phase_us": phases}


def sgemm_floor(quick=False):
    """The matrix-core floor of short SGEMM launches next to the library's SGEMM: bin/sgemm_floor's
    register-only MFMA probe (one wave per SIMD, 0..512 MFMAs per wave, graphs of 50 launches)
    and sgpu_sgemm_opt at 1024^3, 768x1024x1024 and 1023x1025x997 timed the same way."""
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "sgemm_floor")
    log(f"sgemm floor: {exe}")
    r = subprocess.run([exe] + (["--quick"] if quick else []), capture_output=True, text=True, timeout=300)
    sys.stderr.write(r.stderr)
    if r.returncode != 0:
        raise SystemExit(f"sgemm_floor exited {r.returncode}")
    return {"sgemm_floor": json.loads(r.stdout)}


def sgemm_floor_summary():
    """The register-only MFMA kernel with a 1024^3 SGEMM's MFMA count per SIMD (512 per wave)
    next to sgpu_sgemm_opt at 1024^3 and 1023x1025x997, timed the same way in one process
    (bin/sgemm_floor --quick; the full ladder is --sgemm-floor)."""
    try:
        f = sgemm_floor(quick=True)["sgemm_floor"]
    except (OSError, SystemExit, ValueError, subprocess.TimeoutExpired) as e:
        return {"error": str(e)}
    probe = next(r for r in f["mfma"] if r["mfma_per_wave"] == 512)
    sg = {f"{r['M']}x{r['N']}x{r['K']}": r for r in f["sgemm"]}
    k, rg = sg["1024x1024x1024"], sg["1023x1025x997"]
    return {"probe_us": probe["us"],
            "probe_frac_of_peak": round(2 * 1024 ** 3 / probe["us"] / 1e6 / PEAK_FP32_MATRIX_TFLOPS, 4),
            "sgemm_1024_us": k["us"], "sgemm_1024_frac_of_probe": round(probe["us"] / k["us"], 4),
            "ragged_us": rg["us"], "ragged_frac_of_probe": round(probe["us"] / rg["us"], 4),
            "checks": f["checks"]}


def gemv_byname_lm_head():
    """gemv_h launched by name from the qwen_kernels code object at the reference engine's grid
    ((N+7)/8 blocks of 256, qwen_engine.c:265) on the lm_head [151936 x 896], weight copies rotated
    across 600 MB: bin/gemv_test checks it against its CPU golden, then times it."""
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "gemv_test")
    co = os.path.join(ROOT, "switch-l4t-gpu_amd", "build", "qwen_kernels.co")
    try:
        r = subprocess.run([exe, co, "151936", "896", "--h", "--normal", "--rotate", "600", "--json"],
                           capture_output=True, text=True, timeout=180)
        k = json.loads(r.stdout.strip().splitlines()[-1])["kernels"][0]
    except (OSError, ValueError, IndexError, KeyError, subprocess.TimeoutExpired) as e:
        return {"error": str(e)}
    return {"kernel": "gemv_h launched by name", "shape": [151936, 896], "grid": k["grid"], "us": k["us"],
            "gbps": k["gbps"], "frac_hbm": round(k["gbps"] / PEAK_HBM_GBPS, 4), "verdict": k["verdict"]}


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    return oracle


def cpu_gemv_baseline(W, x, reps=3):
    """og_gemv_h (cpu_gemv_h, qwen_engine.c:276-284, serial k order per row) on the lm_head
    [151936 x 896], row-parallel over the host threads (best of `reps`) and on one thread."""
    oracle = _oracle()
    N, K = 151936, 896
    threads = cpu_threads()
    algo = 2.0 * N * K + 4.0 * K + 4.0 * N
    best = 1e9
    for _ in range(reps):
        t = time.perf_counter()
        oracle.gemv_h(W, x, None, K, N, threads)
        best = min(best, time.perf_counter() - t)
    t = time.perf_counter()
    oracle.gemv_h(W, x, None, K, N, 1)
    t1 = time.perf_counter() - t
    return dict(value=round(algo / best / 1e9, 2), unit="GB/s", cores=threads, kind="port",
                sample=f"oracle og_gemv_h on the whole lm_head [151936 x 896] fp16 weights (the GPU leg's W and x), "
                       f"best of {reps} on {threads} threads: {best * 1e3:.1f} ms",
                single_thread={"value": round(algo / t1 / 1e9, 3), "unit": "GB/s", "ms": round(t1 * 1e3, 1)},
                **host_info())


def cpu_decode_baseline(cfg, blob, ids, tokens=4, single_tokens=2):
    """og_qwen_forward (cpu_forward, qwen_engine.c:292-358) on the bench's random-init model:
    positions 0..tokens-1 of the bench prompt, row-parallel GEMVs over the host threads; then
    positions 0..single_tokens-1 again on one thread.  tok/s over those positions."""
    oracle = _oracle()
    ocfg = oracle.qwen_cfg(cfg.V, cfg.C, cfg.NL, cfg.NH, cfg.NKV, cfg.HD, cfg.FC, cfg.CTX, cfg.eps, cfg.theta)
    threads = cpu_threads()
    g = oracle.QwenGolden(ocfg, blob, nthreads=threads)
    t = time.perf_counter()
    for p in range(tokens):
        g.forward(ids[p], p, want_logits=True)
    dt = time.perf_counter() - t
    g1 = oracle.QwenGolden(ocfg, blob, nthreads=1)
    t = time.perf_counter()
    for p in range(single_tokens):
        g1.forward(ids[p], p, want_logits=True)
    dt1 = time.perf_counter() - t
    return dict(value=round(tokens / dt, 3), unit="tok/s", cores=threads, kind="port",
                sample=f"oracle og_qwen_forward, positions 0..{tokens - 1} of the bench's 32-id prompt on the same "
                       f"random-init Qwen2.5-0.5B-architecture weights, logits every position, {threads} threads: "
                       f"{dt:.2f} s",
                single_thread={"value": round(single_tokens / dt1, 3), "unit": "tok/s", "tokens": single_tokens,
                               "s": round(dt1, 2)},
                **host_info())


def cpu_baseline(n, target_s=1.5):
    oracle = _oracle()
    threads = cpu_threads()
    A, B = sgpu.gen_sgemm_inputs(n * n, 42)
    rows = threads
    t = time.perf_counter()
    oracle.sgemm_rows(A, B, n, n, n, 0, rows, threads)
    dt = time.perf_counter() - t
    rows = int(min(n, max(threads, rows * target_s / max(dt, 1e-3))))
    rows -= rows % threads or 0
    rows = max(rows, threads)
    t = time.perf_counter()
    oracle.sgemm_rows(A, B, n, n, n, 0, rows, threads)
    dt = time.perf_counter() - t
    tflops = 2.0 * rows * n * n / dt / 1e12
    return dict(value=tflops, unit="TFLOP/s", cores=threads, kind="port",
                sample=f"oracle og_sgemm_rows (serial k-order fp32, -O2 -ffp-contract=off), rows 0..{rows - 1} "
                       f"of the {n}^3 SGEMM ({2.0 * rows * n * n / 1e9:.1f} GFLOP), {dt:.2f} s on {threads} threads",
                **host_info())


def pmc_probe():
    """One launch each of: add2 over 64 Mi floats (a plain elementwise kernel whose HBM
    traffic is known: 512 MiB read, 256 MiB written -- the counter calibration), the lm_head
    gemv_h and gemv_hh, and ten back-to-back launches each of sgpu_sgemm_opt at 4096^3 and
    1024^3 (sgemm_kwave) and 1023x1025x997 (sgemm_kwave_edge); per-dispatch
    counters are averaged.  Run under `rocprofv3 --pmc FETCH_SIZE`, again with WRITE_SIZE,
    and with the MFMA-busy counters; prints the algorithmic bytes of each launch as one JSON
    line."""
    n = 64 << 20
    a = sgpu.DeviceArray(n)
    b = sgpu.DeviceArray(n)
    c = sgpu.DeviceArray(n)
    for d in (a, b, c):
        d.fill_bytes(0)
    sgpu.synchronize()
    sgpu.call("sgpu_add2", a.ptr, b.ptr, c.ptr, n, None)
    sgpu.synchronize()
    del a, b, c
    N4 = 4096
    A, B = sgpu.gen_sgemm_inputs(N4 * N4, 42)
    dA, dB, dC = sgpu.DeviceArray.from_host(A), sgpu.DeviceArray.from_host(B), sgpu.DeviceArray((N4, N4))
    sgpu.synchronize()
    for _ in range(10):
        sgpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, N4, N4, N4, None)
    sgpu.synchronize()
    del dA, dB, dC
    mids = ((1024, 1024, 1024), (1023, 1025, 997))
    for M, Nm, Km in mids:
        A, B = sgpu.gen_sgemm_inputs(max(M * Km, Km * Nm), 42)
        dA, dB = sgpu.DeviceArray.from_host(A[:M * Km]), sgpu.DeviceArray.from_host(B[:Km * Nm])
        dC = sgpu.DeviceArray((M, Nm))
        sgpu.synchronize()
        for _ in range(10):
            sgpu.call("sgpu_sgemm_opt", dA.ptr, dB.ptr, dC.ptr, M, Nm, Km, None)
        sgpu.synchronize()
        del dA, dB, dC
    N, K = 151936, 896
    W = sgpu.f32_to_f16(sgpu.gen_normal(N * K, 42, 0.0, 0.02)[0])
    dW, dx, dy = sgpu.DeviceArray.from_host(W), sgpu.DeviceArray(K), sgpu.DeviceArray(N)
    dx.fill_bytes(0)
    dxh = sgpu.DeviceArray(K, np.uint16)
    dxh.fill_bytes(0)
    # a 1 GiB read sweep before each GEMV evicts the 256 MB MALL, so neither reads the other's
    # (or the upload's) lines from it
    flush = sgpu.DeviceArray(1 << 28)
    flush.fill_bytes(0)
    fout = sgpu.DeviceArray(1 << 20)
    sgpu.synchronize()
    for fn, xv in (("sgpu_gemv_h", dx), ("sgpu_gemv_hh", dxh)):
        sgpu.call("sgpu_membw_read4", flush.ptr, fout.ptr, (1 << 28) // 4, 1, None, None)
        sgpu.synchronize()
        sgpu.call(fn, dW.ptr, xv.ptr, None, dy.ptr, K, N, None)
        sgpu.synchronize()
    print(json.dumps({"add2_read": 2 * 4 * n, "add2_write": 4 * n,
                      "sgemm_read_min": 2 * 4 * N4 * N4, "sgemm_write": 4 * N4 * N4,
                      **{f"sgemm_{M}x{Nm}x{Km}_read_min": 4 * (M * Km + Km * Nm) for M, Nm, Km in mids},
                      **{f"sgemm_{M}x{Nm}x{Km}_write": 4 * M * Nm for M, Nm, Km in mids},
                      "gemv_h_read": 2 * N * K + 4 * K, "gemv_h_write": 4 * N,
                      "gemv_hh_read": 2 * N * K + 2 * K, "gemv_hh_write": 4 * N}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-decode", action="store_true", help="skip the decode leg")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the SGEMM size sweep and GEMV shape legs (they replay recorded graphs)")
    ap.add_argument("--pmc-probe", action="store_true", help="one launch per measured kernel, for rocprofv3 --pmc")
    ap.add_argument("--decode-only", action="store_true", help="run only the decode leg (for profiling it)")
    ap.add_argument("--sweep-only", action="store_true",
                    help="run only the SGEMM size sweep, host-loop launches (for profiling it)")
    ap.add_argument("--decode-path", choices=["reference", "fused", "graph"], default="graph")
    ap.add_argument("--decode-model", choices=["qwen", "gpt2"], default="qwen",
                    help="model of the --decode-only leg (gpt2: the graph path)")
    ap.add_argument("--decode-floor", action="store_true",
                    help="measure the decode structure's launch and streaming floors and the per-phase "
                         "in-graph times (one JSON line)")
    ap.add_argument("--sgemm-floor", action="store_true",
                    help="measure the matrix-core floor of short SGEMM launches beside sgpu_sgemm_opt (one JSON line)")
    ap.add_argument("--quick", action="store_true", help="fewer repetitions in --decode-floor / --sgemm-floor")
    args = ap.parse_args()
    if args.sgemm_floor:
        sgpu.init(0)
        print(json.dumps(sgemm_floor(args.quick)), flush=True)
        return
    if args.decode_floor:
        sgpu.init(0)
        print(json.dumps(decode_floor(args.quick)), flush=True)
        return
    if args.decode_only:
        sgpu.init(0)
        if args.decode_model == "gpt2":
            dec = bench_gpt2_decode()
            print(json.dumps({"gpt2_decode_tok_s": round(dec["tok_s"], 2), "ms_per_token": round(dec["ms_per_tok"], 4)}))
            return
        path = {"reference": 0, "fused": 1, "graph": 2}[args.decode_path]
        dec = bench_decode(path=path, compare=False)
        print(json.dumps({"decode_tok_s": round(dec["tok_s"], 2), "ms_per_token": round(dec["ms_per_tok"], 4)}))
        return
    if args.sweep_only:
        sgpu.init(0)
        print(json.dumps({"sgemm_sweep": bench_sgemm_sweep(graphs=False)}))
        return
    if args.pmc_probe:
        sgpu.init(0)
        pmc_probe()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (bench.py has no "
              f"multi-GPU path; run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        sys.exit("--steps must be >= 1 and --warmup >= 0")

    sgpu.init(0)
    props = sgpu.device_props(0)
    log(f"device: {props.name.decode()} ({props.arch.decode()}), {props.compute_units} CUs, "
        f"{props.clock_khz / 1e3:.0f} MHz")
    n = 4096
    S = ct.c_int(0)
    member = sgpu.lib().sgpu_sgemm_opt_plan(n, n, n, props.compute_units, ct.byref(S)).decode()
    sg = bench_sgemm(n, args.steps, args.warmup)
    tflops = sg["flops"] * args.steps / sg["wall_s"] / 1e12
    achieved = sg["flops"] / (sg["kernel_ms"] * 1e-3) / 1e12
    log(f"sgpu_sgemm_opt {n}^3: {sg['kernel_ms']:.3f} ms/launch, {achieved:.1f} TFLOP/s kernel, "
        f"{tflops:.1f} TFLOP/s wall, normwise err {sg['err']:.2e}")
    log(f"sgemm steady state: {sg['steady_ms']:.3f} ms/launch over {sg['steady_launches']} launches "
        f"({sg['flops'] / (sg['steady_ms'] * 1e-3) / 1e12:.1f} TFLOP/s); clock settling {sg['settle_launches']} launches")
    gv = bench_gemv_lm_head()
    log(f"gemv_h lm_head: {gv['us']:.1f} us, {gv['gbps']:.0f} GB/s ({gv['gbps'] / PEAK_HBM_GBPS:.1%} of HBM), "
        f"err {gv['err']:.2e}")
    gvh = bench_gemv_lm_head(x16=True)
    log(f"gemv_hh lm_head (fp16 x): {gvh['us']:.1f} us, {gvh['gbps']:.0f} GB/s "
        f"({gvh['gbps'] / PEAK_HBM_GBPS:.1%} of HBM), err {gvh['err']:.2e}")
    cpu_gv = None if args.no_cpu else cpu_gemv_baseline(gv["W"], gv["x"])
    if cpu_gv:
        log(f"cpu gemv_h lm_head: {cpu_gv['value']} GB/s on {cpu_gv['cores']} threads, "
            f"{cpu_gv['single_thread']['value']} GB/s on one")
    del gv["W"], gv["x"], gvh["W"], gvh["x"]
    sweep = gshapes = floor = byname = None
    if not args.no_sweep:
        sweep = bench_sgemm_sweep(cpu=not args.no_cpu)
        log("sgemm sweep (in-graph): " + ", ".join(f"{r['M']}x{r['N']}x{r['K']} {r['tflops']:.1f} TF" for r in sweep))
        gshapes = bench_gemv_shapes(cpu=not args.no_cpu)
        log("gemv shapes (in-graph): " + ", ".join(f"{r['name']} {r['us_in_graph']:.2f} us" for r in gshapes))
        floor = sgemm_floor_summary()
        log(f"sgemm floor: {floor}")
        byname = gemv_byname_lm_head()
        log(f"gemv_h by name at the reference grid: {byname}")
    dec = g2 = cpu_dec = None
    if not args.no_decode:
        dec = bench_decode(keep_blob=not args.no_cpu)
        log(f"decode: {dec['tok_s']:.1f} tok/s ({dec['ms_per_tok']:.3f} ms/token, "
            f"{dec['hbm_floor_frac']:.1%} of the HBM floor)")
        if dec["blob"] is not None:
            cpu_dec = cpu_decode_baseline(dec["cfg"], dec["blob"], dec["ids"])
            log(f"cpu decode: {cpu_dec['value']} tok/s on {cpu_dec['cores']} threads, "
                f"{cpu_dec['single_thread']['value']} tok/s on one")
        dec["blob"] = None
        g2 = bench_gpt2_decode()
        log(f"gpt2 decode: {g2['tok_s']:.1f} tok/s ({g2['ms_per_tok']:.3f} ms/token, "
            f"{g2['hbm_floor_frac']:.1%} of the HBM floor)")
    cpu = None if args.no_cpu else cpu_baseline(n)
    traffic = {}
    if os.path.exists(PROFILE_TRAFFIC):
        traffic = json.load(open(PROFILE_TRAFFIC))
    out = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sg["wall_s"] / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "SGEMM C=A*B M=N=K=4096 fp32 row-major, A,B from srand(42) "
                               "(rand()%2000-1000)/1000, alpha=1 beta=0, sgpu_sgemm_opt (launches the member "
                               f"{member} at this shape)",
                   "M": n, "N": n, "K": n, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MATRIX_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MATRIX_TFLOPS, 4),
                     "kernel": member, "traffic": traffic.get(f"{member}_4096")},
        "cpu_baseline": cpu,
        "steady_state": {"kernel_ms": round(sg["steady_ms"], 4), "launches": sg["steady_launches"],
                         "tflops": round(sg["flops"] / (sg["steady_ms"] * 1e-3) / 1e12, 3),
                         "frac": round(sg["flops"] / (sg["steady_ms"] * 1e-3) / 1e12 / PEAK_FP32_MATRIX_TFLOPS, 4),
                         "clock_settle_s": sg["settle_s"], "clock_settle_launches": sg["settle_launches"]},
        "gemv": {"kernel": "gemv_h (fp16 weights, fp32 x/y)", "shape": [151936, 896],
                 "us_per_call": round(gv["us"], 3), "gbps": round(gv["gbps"], 1),
                 "roofline": {"bound": "hbm", "achieved": round(gv["gbps"], 1), "peak": PEAK_HBM_GBPS,
                              "unit": "GB/s", "frac": round(gv["gbps"] / PEAK_HBM_GBPS, 4),
                              "traffic": traffic.get("gemv_h_lm_head")},
                 "weight_copies_rotated": gv["copies"], "normwise_err": gv["err"], "cpu_baseline": cpu_gv},
        "gemv_hh": {"kernel": "gemv_hh (fp16 weights, fp16 x, fp32 y)", "shape": [151936, 896],
                    "us_per_call": round(gvh["us"], 3), "gbps": round(gvh["gbps"], 1),
                    "roofline": {"bound": "hbm", "achieved": round(gvh["gbps"], 1), "peak": PEAK_HBM_GBPS,
                                 "unit": "GB/s", "frac": round(gvh["gbps"] / PEAK_HBM_GBPS, 4),
                                 "traffic": traffic.get("gemv_hh_lm_head")},
                    "weight_copies_rotated": gvh["copies"], "normwise_err": gvh["err"]},
        "sgemm_sweep": sweep,
        "sgemm_floor": floor,
        "gemv_shapes": gshapes,
        "gemv_byname": byname,
        "decode": None if dec is None else {
            "model": "Qwen2.5-0.5B architecture, random-init N(0,0.02) fp16 weights",
            "tok_s": round(dec["tok_s"], 2), "ms_per_token": round(dec["ms_per_tok"], 4),
            "prompt": dec["prompt"], "generated": dec["generated"],
            "bytes_per_token": dec["bytes_per_token"], "hbm_floor_frac": round(dec["hbm_floor_frac"], 4),
            "path": "fused kernels (5 per layer) replayed as a HIP graph, greedy argmax on the device",
            "prefill_ms": round(dec["prefill_ms"], 3),
            "tok_s_host_argmax_loop": round(dec["host_loop_graph"], 2),
            "tok_s_reference_launch_sequence": round(dec["host_loop_reference"], 2),
            "cpu_baseline": cpu_dec},
        "gpt2_decode": None if g2 is None else {
            "model": "GPT-2 124M architecture, random-init fp32 weights ((frand()-0.5)*0.06)",
            "tok_s": round(g2["tok_s"], 2), "ms_per_token": round(g2["ms_per_tok"], 4),
            "prompt": g2["prompt"], "generated": g2["generated"], "bytes_per_token": g2["bytes_per_token"],
            "hbm_floor_frac": round(g2["hbm_floor_frac"], 4), "prefill_ms": round(g2["prefill_ms"], 3),
            "path": "fused kernels (5 per layer) replayed as a HIP graph, greedy argmax on the device"},
        "sgemm_normwise_err": sg["err"],
        "device": props.name.decode(),
        "host": host_info(),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
