"""On-disk formats written by the engine CLIs, checked without a GPU.

`qwen_engine --write-weights` and `gpt2_engine --write-weights` write the flat weight files
the reference engines load (qwen_engine.c:61-75 written by conv_qwen.py:63-99;
gpt2_engine.c:50-70 written by conv_gpt2.py:47-52 / make_random_bin.py:8-9) and exit before
any device call.  The files must equal, byte for byte, the in-memory models that the GPU
parity tests run, and the loaders must refuse a file of the wrong size with exit status 2
(the reference engines' argument/file error status)."""
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin")


def run(args):
    return subprocess.run(args, capture_output=True, text=True, timeout=300)


def test_qwen_write_weights_is_the_random_model(sg, og, tmp_path):
    f = tmp_path / "qwen.bin"
    r = run([os.path.join(BIN, "qwen_engine"), "--random", "5", "--write-weights", str(f)])
    assert r.returncode == 0, r.stderr
    cfg = sg.qwen_default_cfg()
    blob = np.fromfile(f, np.uint8)
    assert blob.size == 990_162_688
    assert np.array_equal(blob, sg.qwen_random_blob(cfg, seed=5, std=0.02))
    # fp32 RoPE tables follow the fp16 embedding: CTX x HD/2 cos, then sin (qwen_engine.c:61-64,
    # conv_qwen.py:23-27); checked against their closed form
    half, off = cfg.HD // 2, cfg.V * cfg.C * 2
    tabs = blob[off:off + 2 * cfg.CTX * half * 4].view(np.float32).reshape(2, cfg.CTX, half)
    cos, sin = og.rope_tables(cfg.CTX, cfg.HD, cfg.theta)
    assert np.array_equal(tabs[0], cos) and np.array_equal(tabs[1], sin)
    pos = np.arange(cfg.CTX, dtype=np.float64)[:, None]
    ang = pos * cfg.theta ** (-2.0 * np.arange(half) / cfg.HD)
    assert np.array_equal(tabs[0], np.cos(ang).astype(np.float32))


def test_gpt2_write_weights_is_the_random_model(sg, tmp_path):
    f = tmp_path / "gpt2.bin"
    r = run([os.path.join(BIN, "gpt2_engine"), "--random", "5", "--write-weights", str(f)])
    assert r.returncode == 0, r.stderr
    w = np.fromfile(f, np.float32)
    assert w.size == 124_439_808
    want = sg.gpt2_random_weights(sg.gpt2_cfg(), seed=5)
    assert np.array_equal(w, want)
    assert np.abs(w).max() <= 0.03 and abs(float(w.mean())) < 1e-4


def test_round_trip_through_weights_and_bad_sizes(tmp_path):
    """A written GPT-2 file reloads through --weights and is rewritten unchanged; a file of
    the wrong size is refused by either loader with status 2 before the device is touched."""
    exe = os.path.join(BIN, "gpt2_engine")
    a, b = tmp_path / "a.bin", tmp_path / "b.bin"
    assert run([exe, "--random", "9", "--write-weights", str(a)]).returncode == 0
    r = run([exe, "--weights", str(a), "--write-weights", str(b)])
    assert r.returncode == 0, r.stderr
    assert a.read_bytes() == b.read_bytes()
    short = tmp_path / "short.bin"
    short.write_bytes(bytes(4096))
    for name in ("gpt2_engine", "qwen_engine"):
        r = run([os.path.join(BIN, name), "--weights", str(short)])
        assert r.returncode == 2 and "expected" in r.stderr, (name, r.stderr)


def _serial_dot(a, b):
    """The reference golden's serial fp32 sum of fp32 products (gpu_workload.c:97-98)."""
    acc = np.float32(0)
    for p in (a.astype(np.float32) * b.astype(np.float32)):
        acc = np.float32(acc + p)
    return acc


def test_gpu_workload_mismatch_report(sg):
    """The harness's golden-check diagnostics (gpu_workload.c:103-131) on planted errors, host
    only: the first mismatch carries the partial sums over k < 32, 64 and 96, two more follow
    in the short form, one cell per row, and the naive bisect counts every bad cell."""
    r = run([os.path.join(BIN, "gpu_workload"), "--diagnostics-selftest"])
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    n = 256
    A, B = sg.gen_sgemm_inputs(n * n, 42)
    A, B = A.reshape(n, n), B.reshape(n, n)

    def cell(i, j, kend=n):
        return _serial_dot(A[i, :kend], B[:kend, j])

    want = [f"  mismatch [3][7]: got {cell(3, 7) + np.float32(1):.4f} want {cell(3, 7):.4f} "
            f"(k<32:{cell(3, 7, 32):.4f} k<64:{cell(3, 7, 64):.4f} k<96:{cell(3, 7, 96):.4f})",
            f"  mismatch [10][0]: got {cell(10, 0) + np.float32(1):.4f} want {cell(10, 0):.4f}",
            f"  mismatch [11][5]: got {cell(11, 5) + np.float32(1):.4f} want {cell(11, 5):.4f}",
            "sgemm 256: WRONG",
            "sgemm_naive 256: WRONG (6 bad cells)"]
    assert lines == want
