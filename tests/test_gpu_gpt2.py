"""GPT-2 fp32 decode path on the GPU: the support kernels around its GEMVs
(gpt2_kernels.cu:157-268) and the engine's gpu_forward / --fused / gpu_prefill call sequences
(sgpu_gpt2_*, gpt2_engine.c:174-326) against the oracle's cpu_forward (og_gpt2_forward).

Bars: support kernels within fp32 rounding of float64 formulas; engine logits at every
teacher-forced position within 1e-4 of the logit scale with the same argmax, plain and
fused, and the batched prefill's last-row logits likewise; full GPT-2 124M random-init
greedy decode token-identical to the CPU golden for 32 tokens (spec init) and 64 tokens (a
unit-LayerNorm-gain, projections-x4 variant whose greedy continuation does not cycle), and 64 random ids
teacher-forced with every position's logits within 1e-4 of scale (top-1/top-2 gaps printed)."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NT = min(16, os.cpu_count() or 1)
SMALL = dict(V=1000, C=768, NL=2, NH=12, HD=64, FC=3072, CTX=64)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(gpu, a):
    return gpu.DeviceArray.from_host(np.ascontiguousarray(a))


def unit_gain_weights(gpu, cfg, seed):
    """Random-init weights with LayerNorm gains near 1 (so every stage carries signal)."""
    from test_oracle_gpt2 import split

    w = gpu.gpt2_random_weights(gpu.gpt2_cfg(**cfg), seed, 0.03)
    _, _, layers, lnfw, _ = split(w, cfg)
    for L in layers:
        L["ln1w"] += 1.0
        L["ln2w"] += 1.0
        L["fcb"] *= 30.0
    lnfw += 1.0
    return w


def test_layernorm_rows(gpu, og):
    rng = np.random.default_rng(1)
    rows, n = 5, 768
    x = (rng.standard_normal((rows, n)) * 2 + 0.5).astype(np.float32)
    w, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    dx, dw, db, dy = dev(gpu, x), dev(gpu, w), dev(gpu, b), gpu.DeviceArray((rows, n))
    gpu.call("sgpu_layernorm", dx.ptr, dw.ptr, db.ptr, dy.ptr, n, 1e-5, rows, None)
    gpu.synchronize()
    y = dy.to_host()
    for r in range(rows):
        assert np.allclose(y[r], og.layernorm(x[r], w, b, 1e-5), rtol=1e-5, atol=2e-6)


def test_gelu_bias(gpu):
    rng = np.random.default_rng(2)
    n = 3072
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    dx, db = dev(gpu, x), dev(gpu, b)
    gpu.call("sgpu_add_bias", dx.ptr, db.ptr, n, None)
    gpu.call("sgpu_gelu", dx.ptr, dx.ptr, n, None)     # in place, as gpt2_engine.c:236
    gpu.synchronize()
    v = (x + b).astype(np.float64)
    want = 0.5 * v * (1 + np.tanh(0.7978845608 * (v + 0.044715 * v ** 3)))
    assert np.allclose(dx.to_host(), want, rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("T", [1, 3, 100])
def test_attention(gpu, T):
    rng = np.random.default_rng(T)
    q = rng.standard_normal(768).astype(np.float32)
    kc = rng.standard_normal((T, 768)).astype(np.float32)
    vc = rng.standard_normal((T, 768)).astype(np.float32)
    dq, dk, dv = dev(gpu, q), dev(gpu, kc), dev(gpu, vc)
    dsc, dpr, dout = gpu.DeviceArray(T * 12), gpu.DeviceArray(T * 12), gpu.DeviceArray(768)
    gpu.call("sgpu_gpt2_attn_scores", dq.ptr, dk.ptr, dsc.ptr, T, 0.125, None)
    gpu.call("sgpu_gpt2_attn_softmax", dsc.ptr, dpr.ptr, T, None)
    gpu.call("sgpu_gpt2_attn_mix", dpr.ptr, dv.ptr, dout.ptr, T, None)
    gpu.synchronize()
    qh = q.reshape(12, 64).astype(np.float64)
    k = kc.reshape(T, 12, 64).astype(np.float64)
    sc = np.einsum("hd,thd->th", qh, k) * 0.125
    p = np.exp(sc - sc.max(0))
    p /= p.sum(0)
    out = np.einsum("th,thd->hd", p, vc.reshape(T, 12, 64).astype(np.float64)).reshape(768)
    assert np.allclose(dsc.to_host().reshape(T, 12), sc, rtol=1e-5, atol=1e-5)
    assert np.allclose(dpr.to_host().reshape(T, 12), p, rtol=1e-5, atol=1e-7)
    assert np.allclose(dout.to_host(), out, rtol=1e-5, atol=1e-5)


PATHS = {"reference": 0, "reference-fused": 0, "fused": 1, "graph": 2}


@pytest.mark.parametrize("path", sorted(PATHS))
def test_engine_small_teacher_forced(gpu, og, path):
    """Every position's logits against the CPU golden for each launch structure: the
    reference sequence (plain and --fused), five fused kernels per layer, and those replayed
    as one captured graph (position in device memory)."""
    cfg = SMALL
    fused = path == "reference-fused"
    w = unit_gain_weights(gpu, cfg, 23)
    eng = gpu.Gpt2Engine(gpu.gpt2_cfg(**cfg), w, PATHS[path])
    gold = og.Gpt2Golden(og.gpt2_cfg(**cfg), w, NT)
    ids = [int(v) for v in np.random.default_rng(7).integers(0, cfg["V"], 30)]
    for p, t in enumerate(ids):
        got = eng.forward(t, p, True, fused).copy()
        want = gold.forward(t, p)
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 1e-4 * scale, (p, np.abs(got - want).max(), scale)
        assert int(np.argmax(got)) == og.argmax(want)
    eng.close()


def test_engine_long_context_fused(gpu, og):
    """400 teacher-forced positions on the fused path: past 256 cached positions the attention
    cuts each head's cache into chunks and combines their partials; logits track the CPU
    golden at every checked position."""
    cfg = dict(SMALL, NL=1, CTX=400)
    w = unit_gain_weights(gpu, cfg, 29)
    eng = gpu.Gpt2Engine(gpu.gpt2_cfg(**cfg), w, PATHS["fused"])
    gold = og.Gpt2Golden(og.gpt2_cfg(**cfg), w, NT)
    ids = [int(v) for v in np.random.default_rng(8).integers(0, cfg["V"], cfg["CTX"])]
    for p, t in enumerate(ids):
        check = p % 25 == 24 or p >= cfg["CTX"] - 2
        got = eng.forward(t, p, check, 0)
        want = gold.forward(t, p, check)
        if not check:
            continue
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 1e-4 * scale, (p, np.abs(got - want).max(), scale)
        assert int(np.argmax(got)) == og.argmax(want)
    eng.close()


@pytest.mark.parametrize("path", ["reference", "fused", "graph"])
def test_engine_small_generate(gpu, og, path):
    """sgpu_gpt2_generate (device-side argmax and embedding on the fused/graph paths) gives the
    CPU golden's greedy ids, and a second call restarts at position 0."""
    cfg = SMALL
    w = unit_gain_weights(gpu, cfg, 31)
    eng = gpu.Gpt2Engine(gpu.gpt2_cfg(**cfg), w, PATHS[path])
    prompt = [int(v) for v in np.random.default_rng(9).integers(0, cfg["V"], 7)]
    got = eng.generate(prompt, 16)
    gold = og.Gpt2Golden(og.gpt2_cfg(**cfg), w, NT)
    for p, t in enumerate(prompt):
        ref = gold.forward(t, p, p == len(prompt) - 1)
    want = [og.argmax(ref)]
    for g in range(16):
        ref = gold.forward(want[-1], len(prompt) + g)
        want.append(og.argmax(ref))
    assert got.tolist() == want
    assert eng.generate(prompt, 16).tolist() == want
    eng.close()


def test_engine_full_generate_graph_token_identical(gpu, og):
    """Full GPT-2 124M random init, graph path, on-device greedy loop: the 8-id deterministic
    prompt and 32 generated positions; the CPU golden, fed the same ids, picks the same argmax
    at every position."""
    cfg = gpu.gpt2_cfg()
    w = gpu.gpt2_random_weights(cfg, 42, 0.03)
    eng = gpu.Gpt2Engine(cfg, w, 2)
    prompt = [(i * 7919 + 42) % cfg.V for i in range(8)]       # gpt2_engine.c deterministic prompt
    got = eng.generate(prompt, 32).tolist()
    gold = og.Gpt2Golden(og.gpt2_cfg(), w, NT)
    seq = prompt + got
    for p in range(8 + 32):
        ref = gold.forward(seq[p], p, p >= 7)
        if p >= 7:
            assert og.argmax(ref) == seq[p + 1], (p, og.argmax(ref), seq[p + 1])
    eng.close()


def test_engine_batched_prefill(gpu, og):
    """gpu_prefill fills the cache through gemv_multi; decoding on from it must match the
    sequential CPU golden at every later position."""
    cfg = SMALL
    w = unit_gain_weights(gpu, cfg, 29)
    eng = gpu.Gpt2Engine(gpu.gpt2_cfg(**cfg), w)
    gold = og.Gpt2Golden(og.gpt2_cfg(**cfg), w, NT)
    ids = [int(v) for v in np.random.default_rng(8).integers(0, cfg["V"], 20)]
    got = eng.prefill(ids).copy()
    for p, t in enumerate(ids):
        want = gold.forward(t, p, p == len(ids) - 1)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 1e-4 * scale
    nxt = int(np.argmax(got))
    for p in range(len(ids), len(ids) + 8):
        g = eng.forward(nxt, p).copy()
        c = gold.forward(nxt, p)
        assert np.abs(g - c).max() <= 1e-4 * np.abs(c).max()
        assert int(np.argmax(g)) == og.argmax(c)
        nxt = int(np.argmax(g))
    eng.close()


def test_engine_full_greedy_token_identical(gpu, og):
    cfg = gpu.gpt2_cfg()
    say("building GPT-2 124M random weights")
    w = gpu.gpt2_random_weights(cfg, 42, 0.03)
    eng = gpu.Gpt2Engine(cfg, w)
    gold = og.Gpt2Golden(og.gpt2_cfg(), w, NT)
    tokens = [(i * 7919 + 42) % cfg.V for i in range(8)]       # gpt2_engine.c deterministic prompt
    n_total = 8 + 32
    for p in range(n_total):
        want_logits = p >= 7
        got = eng.forward(tokens[p], p, want_logits)
        ref = gold.forward(tokens[p], p, want_logits)
        if not want_logits:
            continue
        g_tok, c_tok = int(np.argmax(got)), og.argmax(ref)
        assert g_tok == c_tok, (p, g_tok, c_tok)
        assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
        if len(tokens) < n_total:
            tokens.append(g_tok)
    eng.close()


# ---- full-size parity that does not reduce to a few embeddings ----
# The spec init draws the LayerNorm gains like every other tensor ((frand() - 0.5) * 0.06), so
# each layer's output is scaled by ~0.03 and the residual stream is dominated by the current
# token's embedding (with the tied lm_head, the current token's own logit).  As for the Qwen
# engine: the spec model teacher-forced over 64 seeded random ids, and a variant decoded
# free-running: LayerNorm gains 1 + their spec value and the four projection matrices (qkv,
# attention out, fc, proj) at 4x the spec amplitude.  Measured on the 8-id prompt (GPU
# reference path against the CPU golden, 64 greedy tokens): unit gains alone give 6 distinct
# tokens in 41; projections x4, 46 of 64 with the logits within 5.5e-6 of scale and every
# top-1/top-2 gap at least 900x the GPU/CPU difference.
FULL = dict(V=50257, C=768, NL=12, NH=12, HD=64, FC=3072, CTX=1024)


def check_position(p, got, ref, gaps, stats):
    """Logits within 1e-4 (fp32 weights) of the logit scale; the argmax equal unless the reference's margin of
    its top token over the GPU's pick is within 4x this position's RMS logit error (a near-tie,
    counted and printed).  The RMS, not the largest error, sets the bar: a flip is always
    within twice the largest error of the two logits involved, so only an outlier error on
    exactly those two logits can flip a wider margin, and that fails the test."""
    err = np.abs(got.astype(np.float64) - ref)
    stats["worst"] = max(stats["worst"], float(err.max() / np.abs(ref).max()))
    assert err.max() <= 1e-4 * np.abs(ref).max(), (p, float(err.max()), float(np.abs(ref).max()))
    top2 = np.sort(ref)[-2:]
    gaps.append(float(top2[1] - top2[0]))
    g_tok, c_tok = int(np.argmax(got)), int(np.argmax(ref))
    if g_tok != c_tok:
        rms = float(np.sqrt(np.mean(err * err)))
        margin = float(ref[c_tok] - ref[g_tok])
        stats.setdefault("flips", []).append((p, c_tok, g_tok, margin, rms))
        assert margin <= 4 * rms, (p, g_tok, c_tok, margin, rms)
        stats["ties"] += 1
    return g_tok


@pytest.fixture(scope="module")
def full_spec(gpu, og):
    say("GPT-2 124M spec model: weights and 64 golden positions")
    w = gpu.gpt2_random_weights(gpu.gpt2_cfg(), 42, 0.03)
    ids = [int(v) for v in np.random.default_rng(64).integers(0, FULL["V"], 64)]
    gold = og.Gpt2Golden(og.gpt2_cfg(), w, NT)
    return w, ids, np.stack([gold.forward(t, p) for p, t in enumerate(ids)])


@pytest.mark.parametrize("path", ["reference", "graph"])
def test_engine_full_teacher_forced(gpu, full_spec, path):
    """GPT-2 124M (spec init), 64 random ids teacher-forced: every position's logits against
    the CPU golden, on the reference launch sequence and on the replayed graph."""
    w, ids, logits = full_spec
    eng = gpu.Gpt2Engine(gpu.gpt2_cfg(), w, {"reference": 0, "graph": 2}[path])
    gaps, stats = [], {"worst": 0.0, "ties": 0}
    for p, t in enumerate(ids):
        check_position(p, eng.forward(t, p, True).copy(), logits[p], gaps, stats)
    eng.close()
    say(f"{path}: 64 teacher-forced positions, worst logit error {stats['worst']:.2e} of scale, "
        f"min top-1/top-2 gap {min(gaps):.3e}, median {np.median(gaps):.3e}, near-ties {stats['ties']} {stats.get('flips', [])}")
    assert stats["ties"] <= 2


@pytest.fixture(scope="module")
def full_variant(gpu, og):
    """LayerNorm gains 1 + their spec value, projections x4; the 8-id deterministic prompt;
    the CPU golden's own greedy continuation of 64 tokens and the logits it took each one from."""
    from test_oracle_gpt2 import split

    say("GPT-2 124M rich variant: weights and the golden's greedy run")
    w = gpu.gpt2_random_weights(gpu.gpt2_cfg(), 42, 0.03)
    _, _, layers, lnfw, _ = split(w, FULL)
    for L in layers:
        L["ln1w"] += 1.0
        L["ln2w"] += 1.0
        for k in ("qkvw", "aow", "fcw", "projw"):
            L[k] *= 4.0
    lnfw += 1.0
    prompt = [(i * 7919 + 42) % FULL["V"] for i in range(8)]     # gpt2_engine.c deterministic prompt
    gold = og.Gpt2Golden(og.gpt2_cfg(), w, NT)
    seq, logits = list(prompt), []
    for p in range(8 + 64):
        ref = gold.forward(seq[p], p, p >= 7)
        if p >= 7:
            logits.append(ref)
            if len(seq) < 8 + 65:
                seq.append(og.argmax(ref))
    return w, prompt, seq[8:], np.stack(logits)


@pytest.mark.parametrize("path", ["reference", "graph"])
def test_engine_full_variant_greedy(gpu, full_variant, path):
    """Free-running greedy decode on the rich variant: 64 tokens token-identical to the CPU
    golden's own greedy run, which does not cycle (at least 24 distinct tokens of 64)."""
    w, prompt, want, logits = full_variant
    distinct = len(set(want[:64]))
    say(f"golden greedy continuation: {want[:12]} ..., {distinct} distinct of 64")
    assert distinct >= 24
    eng = gpu.Gpt2Engine(gpu.gpt2_cfg(), w, {"reference": 0, "graph": 2}[path])
    if path == "graph":
        got = eng.generate(prompt, 64).tolist()
        assert got == want[:65], next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)
    else:
        gaps, stats = [], {"worst": 0.0, "ties": 0}
        seq = list(prompt)
        for p in range(8 + 64):
            out = eng.forward(seq[p], p, p >= 7)
            if p >= 7:
                tok = check_position(p, out.copy(), logits[p - 7], gaps, stats)
                assert tok == want[p - 7], (p, tok, want[p - 7])
                seq.append(tok)
        say(f"reference path: 64 greedy tokens identical, worst logit error {stats['worst']:.2e}, "
            f"min top-1/top-2 gap {min(gaps):.3e}")
    eng.close()


def test_engine_cli_json(gpu):
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "gpt2_engine")
    runs = {}
    for extra in ([], ["--fused"], ["--batch-prefill"], ["--path", "fused"], ["--path", "graph"]):
        out = subprocess.run([exe, "--random", "5", "--gen", "5", "--json"] + extra,
                             capture_output=True, text=True, timeout=300)
        assert out.returncode == 0, out.stderr
        d = json.loads(out.stdout.strip().splitlines()[-1])
        assert d["done"] and d["prompt"] == 8 and d["tok_s"] > 0
        runs[" ".join(extra)] = d["ids"]
    # the device-side greedy loop emits the same ids as the host loop (no EOT in 5 steps)
    assert runs["--path graph"] == runs[""][:len(runs["--path graph"])]


# ---- the CLI's own self-test (--selftest / --debug, gpt2_engine.c:474-535) ----
TRACE_RE = r"trace p0 L(\d+): max\|d\|=([0-9.]+) \(\|gpu\|~([0-9.]+)\)"


def check_selftest_output(text, NL):
    import re

    traces = re.findall(TRACE_RE, text)
    assert [int(t[0]) for t in traces] == list(range(NL)), text[-2000:]
    for layer, d, g in traces:
        assert float(d) <= 1e-4 * max(float(g), 1.0), (layer, d, g)
    assert "SELFTEST: PASS" in text and "MATCH" in text, text[-2000:]
    assert text.count("top-5 ids:") == 2


STAGE_RE = r"^    ([gc])\.(\w+)\s+first4=(\S+) (\S+) (\S+) (\S+) sum=(\S+)$"


def stage_lines(text):
    """{("g"|"c", stage): (first4, sum)} from the --debug stage lines (format of the
    reference's prvec / gprvec)."""
    import re

    out = {}
    for m in re.finditer(STAGE_RE, text, re.M):
        v = [float(x) for x in m.groups()[2:]]
        out[(m.group(1), m.group(2))] = (v[:4], v[4])
    return out


def check_stages_agree(st, tags, tol):
    """The GPU's and the CPU's printed values of each stage both print (3 decimals)."""
    for tag in tags:
        (g4, gs), (c4, cs) = st[("g", tag)], st[("c", tag)]
        for a, b in zip(g4 + [gs], c4 + [cs]):
            assert abs(a - b) <= tol * max(abs(b), 1.0) + 2e-3, (tag, g4, gs, c4, cs)


@pytest.mark.parametrize("extra", [[], ["--fused"], ["--batch-prefill"], ["--path", "graph"]])
def test_cli_selftest(gpu, extra, tmp_path):
    """bin/gpt2_engine --selftest 4 on the full random-init model (fp32 weights): the per-layer
    residual trace at position 0 and the logits at position 3 against the program's own serial
    CPU forward, on the chosen launch form, then a normal run."""
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "gpt2_engine")
    say(f"gpt2_engine --selftest 4 {' '.join(extra)}")
    out = subprocess.run([exe, "--random", "3", "--selftest", "4", "--gen", "4"] + extra,
                         capture_output=True, text=True, timeout=600, cwd=tmp_path)
    assert out.returncode == 0, out.stderr[-2000:]
    check_selftest_output(out.stdout, 12)
    assert ("[batched]" in out.stdout) == ("--batch-prefill" in extra)
    assert "ENGINE_DONE" in out.stdout


def test_forward_stages(gpu):
    """sgpu_gpt2_forward_stages: the reference's twelve layer-0 stages in launch order (plain
    and fused GEMVs), the last one bit-identical to the layer trace of the same launch
    sequence; at position 0 every head's softmax is exactly 1 and its output is its v."""
    cfg = gpu.gpt2_cfg()
    w = gpu.gpt2_random_weights(cfg, 21, 0.03)
    eng = gpu.Gpt2Engine(cfg, w, 0)
    for fused in (False, True):
        logits_s, st = eng.forward_stages(7, 0, fused)
        logits_s = logits_s.copy()
        names = [t for t, _ in st]
        assert names == ["ln1", "qkv", "scores", "probs", "attnout", "ao", "res1", "ln2", "fc", "gelu", "proj",
                         "res2"]
        v = dict(st)
        C, NH, FC = cfg.C, cfg.NH, cfg.FC
        assert [len(v[k]) for k in names] == [C, 3 * C, NH, NH, C, C, C, C, FC, FC, C, C]
        assert np.array_equal(v["probs"], np.ones(NH, np.float32))
        assert np.array_equal(v["attnout"], v["qkv"][2 * C:])
        logits_t, trace = eng.forward_trace(7, 0, fused)
        assert np.array_equal(v["res2"], trace[0]) and np.array_equal(logits_s, logits_t)
    eng.close()


def test_cli_selftest_debug(gpu, tmp_path):
    """--debug adds the layer-0 stage lines, the GPU's (g.*, the reference launch sequence)
    before the CPU forward's (c.*), agreeing where both print a stage, and writes both layer
    traces."""
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "gpt2_engine")
    say("gpt2_engine --selftest 2 --debug")
    out = subprocess.run([exe, "--random", "4", "--selftest", "2", "--debug", "--gen", "1"],
                         capture_output=True, text=True, timeout=600, cwd=tmp_path)
    assert out.returncode == 0, out.stderr[-2000:]
    check_selftest_output(out.stdout, 12)
    for tag in ("embed", "ln1", "qkv", "ao", "res1", "ln2", "fc", "gelu", "proj", "res2"):
        assert f"c.{tag}" in out.stdout
    st = stage_lines(out.stdout)
    assert all(("g", t) in st for t in ("ln1", "qkv", "scores", "probs", "attnout", "ao", "res1", "ln2", "fc", "gelu", "proj", "res2")), sorted(st)
    assert out.stdout.index("g.ln1") < out.stdout.index("c.ln1")
    check_stages_agree(st, ("ln1", "qkv", "ao", "res1", "ln2", "fc", "gelu", "proj", "res2"), 1e-4)
    g = np.fromfile(tmp_path / "trace_g.bin", np.float32)
    c = np.fromfile(tmp_path / "trace_c.bin", np.float32)
    assert g.size == c.size == 12 * 768
    assert np.abs(g - c).max() <= 1e-4 * max(np.abs(g).max(), 1.0)


def test_forward_trace_is_the_reference_forward(gpu):
    """sgpu_gpt2_forward_trace computes what the reference path computes, bit for bit (plain
    and --fused launch forms), on an engine of any path."""
    c = gpu.gpt2_cfg(V=1000, NL=2, CTX=64)
    w = gpu.gpt2_random_weights(c, seed=21)
    ref = gpu.Gpt2Engine(c, w, gpu.GPT2_PATH_REFERENCE)
    tr_eng = gpu.Gpt2Engine(c, w, gpu.GPT2_PATH_GRAPH)
    for fused in (False, True):
        for p, t in enumerate([3, 999, 42, 7]):
            want = ref.forward(t, p, fused=fused).copy()
            got, trace = tr_eng.forward_trace(t, p, fused=fused)
            assert np.array_equal(got, want), (fused, p)
            assert trace.shape == (2, 768) and np.all(np.isfinite(trace))
    ref.close()
    tr_eng.close()
