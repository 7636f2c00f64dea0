"""Qwen2.5 decode path on the GPU: the support kernels each GEMV feeds (qwen_kernels.cu:72-189)
and the engine's per-position forward (sgpu_qwen_forward, the gpu_forward sequence of
qwen_engine.c:205-269) against the oracle's cpu_forward (og_qwen_forward).

Bars: support kernels within fp32 rounding of float64 formulas; engine logits at every
teacher-forced position within 1e-4 of the logit scale with the same argmax; full
Qwen2.5-0.5B-architecture random-init model: greedy decode token-identical to the CPU golden
for 64 tokens after a 32-token prompt (spec init, and a unit-norm-gain, projections-x2 variant whose greedy
continuation does not cycle, 24+ distinct tokens), and 64 random ids teacher-forced with every position's logits
within 1e-3 of scale and the same argmax (top-1/top-2 gaps printed)."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NT = min(16, os.cpu_count() or 1)
SMALL = dict(V=512, C=128, NL=2, NH=4, NKV=2, HD=32, FC=256, CTX=64)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(gpu, a):
    return gpu.DeviceArray.from_host(np.ascontiguousarray(a))


def test_rmsnorm(gpu, og):
    rng = np.random.default_rng(1)
    rows, n = 3, 896
    x = rng.standard_normal((rows, n)).astype(np.float32)
    w = (rng.standard_normal(n) * 0.5).astype(np.float16).view(np.uint16)
    dx, dw, dy = dev(gpu, x), dev(gpu, w), gpu.DeviceArray((rows, n))
    gpu.call("sgpu_rmsnorm", dx.ptr, dw.ptr, dy.ptr, n, 1e-6, rows, None)
    gpu.synchronize()
    y = dy.to_host()
    for r in range(rows):
        assert np.allclose(y[r], og.rms(x[r], w, 1e-6), rtol=2e-6, atol=1e-7)


def test_rope(gpu, og):
    rng = np.random.default_rng(2)
    T, H, HD, pos0, ctx = 3, 14, 64, 5, 64
    c, s = og.rope_tables(ctx, HD, 1e6)
    x = rng.standard_normal((T, H, HD)).astype(np.float32)
    dx, dc, ds = dev(gpu, x), dev(gpu, c), dev(gpu, s)
    gpu.call("sgpu_rope", dx.ptr, dc.ptr, ds.ptr, T, H, HD, pos0, None)
    gpu.synchronize()
    got = dx.to_host()
    a, b = x[..., :HD // 2].astype(np.float64), x[..., HD // 2:].astype(np.float64)
    cc, ss = c[pos0:pos0 + T][:, None, :].astype(np.float64), s[pos0:pos0 + T][:, None, :].astype(np.float64)
    want = np.concatenate([a * cc - b * ss, a * ss + b * cc], axis=-1)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


def test_swiglu_add2(gpu):
    rng = np.random.default_rng(3)
    n = 4864
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    dg, du, dy = dev(gpu, g), dev(gpu, u), gpu.DeviceArray(n)
    gpu.call("sgpu_swiglu", dg.ptr, du.ptr, dy.ptr, n, None)
    gpu.call("sgpu_add2", dg.ptr, du.ptr, du.ptr, n, None)    # in place, as qwen_engine.c:244
    gpu.synchronize()
    g64 = g.astype(np.float64)
    assert np.allclose(dy.to_host(), g64 / (1 + np.exp(-g64)) * u, rtol=1e-6, atol=1e-7)
    assert np.array_equal(du.to_host(), g + u)


@pytest.mark.parametrize("T", [1, 2, 65, 300])
def test_attention_kernels(gpu, T):
    rng = np.random.default_rng(T)
    NH, NKV, HD = 14, 2, 64
    KV = NKV * HD
    q = rng.standard_normal(NH * HD).astype(np.float32)
    kc = rng.standard_normal((T, KV)).astype(np.float32)
    vc = rng.standard_normal((T, KV)).astype(np.float32)
    dq, dk, dv = dev(gpu, q), dev(gpu, kc), dev(gpu, vc)
    dsc, dpr, dout = gpu.DeviceArray(T * NH), gpu.DeviceArray(T * NH), gpu.DeviceArray(NH * HD)
    gpu.call("sgpu_attn_scores_gqa", dq.ptr, dk.ptr, dsc.ptr, T, 0.125, NH, KV, HD, None)
    gpu.call("sgpu_attn_softmax", dsc.ptr, dpr.ptr, T, NH, None)
    gpu.call("sgpu_attn_mix_gqa", dpr.ptr, dv.ptr, dout.ptr, T, NH, KV, HD, None)
    gpu.synchronize()
    g = np.arange(NH) // (NH // NKV)
    qh = q.reshape(NH, HD).astype(np.float64)
    k = kc.reshape(T, NKV, HD).astype(np.float64)[:, g, :]         # [T, NH, HD]
    sc = np.einsum("hd,thd->th", qh, k) * 0.125
    p = np.exp(sc - sc.max(0))
    p /= p.sum(0)
    v = vc.reshape(T, NKV, HD).astype(np.float64)[:, g, :]
    out = np.einsum("th,thd->hd", p, v)
    assert np.allclose(dsc.to_host().reshape(T, NH), sc, rtol=1e-5, atol=1e-5)
    assert np.allclose(dpr.to_host().reshape(T, NH), p, rtol=1e-5, atol=1e-7)
    assert np.allclose(dout.to_host().reshape(NH, HD), out, rtol=1e-5, atol=1e-5)
    if T == 1:   # one position: softmax is exactly 1, the mix returns v bit for bit
        assert np.array_equal(dpr.to_host(), np.ones(NH, np.float32))
        assert np.array_equal(dout.to_host().reshape(NH, HD), vc.reshape(NKV, HD)[g])


PATHS = {"reference": 0, "fused": 1, "graph": 2}


@pytest.mark.parametrize("path", sorted(PATHS))
@pytest.mark.parametrize("std", [0.02, 0.15])
def test_engine_small_teacher_forced(gpu, og, std, path):
    """Every position's logits against the CPU golden, for each launch structure (the graph
    path replays one captured graph at every position, with eager launches between)."""
    cfg = SMALL
    blob = gpu.qwen_random_blob(gpu.qwen_cfg(**cfg), seed=21, std=std)
    eng = gpu.QwenEngine(gpu.qwen_cfg(**cfg), blob, PATHS[path])
    gold = og.QwenGolden(og.qwen_cfg(**cfg), blob, NT)
    ids = [int(v) for v in np.random.default_rng(4).integers(0, cfg["V"], 40)]
    for p, t in enumerate(ids):
        got = eng.forward(t, p).copy()
        want = gold.forward(t, p)
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 1e-4 * scale, (p, np.abs(got - want).max(), scale)
        assert int(np.argmax(got)) == og.argmax(want)
    eng.close()


def wo_offset(c, layer):
    """Half-index of layer `layer`'s o-projection weights in the flat file (qwen_engine.c:61-75:
    embedding, RoPE tables, then per layer in_ln, qkv W, qkv b, o W, ...)."""
    qkv = c["C"] + 2 * c["NKV"] * c["HD"]
    base = (c["V"] * c["C"] * 2 + 2 * c["CTX"] * (c["HD"] // 2) * 4) // 2
    lstride = c["C"] + qkv * c["C"] + qkv + c["C"] * c["C"] + c["C"] + 2 * c["FC"] * c["C"] + c["C"] * c["FC"]
    return base + layer * lstride + c["C"] + qkv * c["C"] + qkv


@pytest.mark.parametrize("path", sorted(PATHS))
def test_engine_exponent31_weights(gpu, og, path):
    """fp16 codes with exponent 31 in the o projection (the reference's h2f decodes them to the
    finite +-2^16(1+m/1024); the hardware conversion gives inf/NaN): every launch structure
    matches the CPU golden, teacher-forced, including the fused attention + o projection."""
    cfg = SMALL
    blob = gpu.qwen_random_blob(gpu.qwen_cfg(**cfg), seed=23, std=0.15)
    h = blob.view(np.uint16)
    o = wo_offset(cfg, 0)
    C, HD = cfg["C"], cfg["HD"]
    for r, k, code in ((5, 0, 0x7C00), (5, HD + 3, 0xFC01), (C - 1, C - 1, 0x7C10), (17, 2 * HD, 0xFFFF)):
        h[o + r * C + k] = code
    eng = gpu.QwenEngine(gpu.qwen_cfg(**cfg), blob, PATHS[path])
    gold = og.QwenGolden(og.qwen_cfg(**cfg), blob, NT)
    ids = [int(v) for v in np.random.default_rng(8).integers(0, cfg["V"], 12)]
    for p, t in enumerate(ids):
        got = eng.forward(t, p).copy()
        want = gold.forward(t, p)
        assert np.all(np.isfinite(want)) and np.all(np.isfinite(got)), p
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 1e-4 * scale, (p, np.abs(got - want).max(), scale)
    eng.close()


@pytest.mark.parametrize("path", sorted(PATHS))
def test_engine_exponent31_norm_gains(gpu, og, path):
    """fp16 codes with exponent 31 and subnormal codes in layer 0's RMSNorm gains (in_ln ahead
    of the qkv projection, post_ln ahead of gate|up).  The fused prologues convert gains in
    hardware; an exponent-31 gain makes every row sum non-finite there, and those rows are
    recomputed with the reference's exact decode (finite +-2^16(1+m/1024); subnormals read as
    0).  Every launch structure matches the CPU golden, teacher-forced."""
    cfg = SMALL
    blob = gpu.qwen_random_blob(gpu.qwen_cfg(**cfg), seed=29, std=0.15)
    h = blob.view(np.uint16)
    C = cfg["C"]
    qkv = C + 2 * cfg["NKV"] * cfg["HD"]
    in_ln = (cfg["V"] * C * 2 + 2 * cfg["CTX"] * (cfg["HD"] // 2) * 4) // 2
    post_ln = in_ln + C + qkv * C + qkv + C * C
    for off, k, code in ((in_ln, 3, 0x7C00), (in_ln, C - 1, 0x0001), (post_ln, 5, 0xFC02), (post_ln, 7, 0x83FF)):
        h[off + k] = code
    eng = gpu.QwenEngine(gpu.qwen_cfg(**cfg), blob, PATHS[path])
    gold = og.QwenGolden(og.qwen_cfg(**cfg), blob, NT)
    ids = [int(v) for v in np.random.default_rng(9).integers(0, cfg["V"], 12)]
    for p, t in enumerate(ids):
        got = eng.forward(t, p).copy()
        want = gold.forward(t, p)
        assert np.all(np.isfinite(want)) and np.all(np.isfinite(got)), p
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 1e-4 * scale, (p, np.abs(got - want).max(), scale)
    eng.close()


# Long teacher-forced runs on the fused path, head dims 32 and 128: the attention kernel's
# score and mix loops take several passes past 64 (32) positions per pass, past 256 positions
# a head's cache is cut into chunks whose partials are combined, and past 7936 the chunk count
# stays at 32 (the 8192-position case runs the whole cache);
# the shapes differ from the 0.5B model's (HD 64); logits must track the CPU golden throughout.
LONG = [dict(V=300, C=128, NL=1, NH=4, NKV=2, HD=32, FC=256, CTX=320, n=300),
        dict(V=300, C=256, NL=1, NH=2, NKV=1, HD=128, FC=512, CTX=300, n=300),
        dict(V=64, C=64, NL=1, NH=2, NKV=1, HD=32, FC=64, CTX=8192, n=8192)]


@pytest.mark.parametrize("case", LONG, ids=["hd32", "hd128", "ctx8192"])
def test_engine_long_context_fused(gpu, og, case):
    cfg = {k: v for k, v in case.items() if k != "n"}
    blob = gpu.qwen_random_blob(gpu.qwen_cfg(**cfg), seed=41, std=0.15)
    eng = gpu.QwenEngine(gpu.qwen_cfg(**cfg), blob, PATHS["fused"])
    gold = og.QwenGolden(og.qwen_cfg(**cfg), blob, NT)
    ids = [int(v) for v in np.random.default_rng(6).integers(0, cfg["V"], case["n"])]
    for p, t in enumerate(ids):
        check = p % (10 if case["n"] < 1000 else 257) == 9 or p >= case["n"] - 3
        got = eng.forward(t, p, check)
        want = gold.forward(t, p, check)
        if not check:
            continue
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 1e-4 * scale, (p, np.abs(got - want).max(), scale)
        assert int(np.argmax(got)) == og.argmax(want)
    eng.close()


# Batched prefill (sgpu_qwen_prefill): the last prompt row's logits, then five decoded
# positions that read the cache the prefill wrote, against the CPU golden run position by
# position.  Prompts past 512 rows are prefilled in chunks that attend to earlier chunks
# through the cache.
PREFILL = [dict(cfg=SMALL, T=1), dict(cfg=SMALL, T=7), dict(cfg=SMALL, T=40),
           dict(cfg=dict(V=300, C=128, NL=2, NH=4, NKV=2, HD=32, FC=256, CTX=1100), T=1030),
           dict(cfg=dict(V=300, C=256, NL=1, NH=2, NKV=1, HD=128, FC=512, CTX=600), T=520)]


@pytest.mark.parametrize("case", PREFILL, ids=["t1", "t7", "t40", "chunked-hd32", "chunked-hd128"])
def test_engine_prefill_matches_golden(gpu, og, case):
    cfg, T = case["cfg"], case["T"]
    say(f"qwen prefill T={T} cfg={cfg}")
    blob = gpu.qwen_random_blob(gpu.qwen_cfg(**cfg), seed=51, std=0.15)
    eng = gpu.QwenEngine(gpu.qwen_cfg(**cfg), blob, PATHS["fused"])
    gold = og.QwenGolden(og.qwen_cfg(**cfg), blob, NT)
    ids = [int(v) for v in np.random.default_rng(T).integers(0, cfg["V"], T + 5)]
    got = eng.prefill(ids[:T]).copy()
    for p in range(T):
        want = gold.forward(ids[p], p, p == T - 1)
    rows = [(T - 1, got, want)]
    for p in range(T, T + 5):
        rows.append((p, eng.forward(ids[p], p, True).copy(), gold.forward(ids[p], p, True)))
    for p, g, w in rows:
        scale = np.abs(w).max()
        assert np.abs(g - w).max() <= 1e-4 * scale, (p, np.abs(g - w).max(), scale)
        assert int(np.argmax(g)) == og.argmax(w), p
    eng.close()


def test_engine_prefill_rejects_bad_ids(gpu):
    cfg = SMALL
    eng = gpu.QwenEngine(gpu.qwen_cfg(**cfg), gpu.qwen_random_blob(gpu.qwen_cfg(**cfg), seed=3), PATHS["fused"])
    with pytest.raises(gpu.SgpuError):
        eng.prefill([1, cfg["V"]])
    with pytest.raises(gpu.SgpuError):
        eng.prefill([1] * (cfg["CTX"] + 1))
    eng.close()


@pytest.mark.parametrize("path", ["reference", "graph"])
def test_engine_small_generate(gpu, og, path):
    """sgpu_qwen_generate (on-device argmax loop for the graph path) gives the CPU golden's
    greedy ids."""
    cfg = SMALL
    blob = gpu.qwen_random_blob(gpu.qwen_cfg(**cfg), seed=33, std=0.15)
    eng = gpu.QwenEngine(gpu.qwen_cfg(**cfg), blob, PATHS[path])
    prompt = [int(v) for v in np.random.default_rng(5).integers(0, cfg["V"], 9)]
    got = eng.generate(prompt, 20)
    gold = og.QwenGolden(og.qwen_cfg(**cfg), blob, NT)
    for p, t in enumerate(prompt):
        ref = gold.forward(t, p, p == len(prompt) - 1)
    want = [og.argmax(ref)]
    for g in range(20):
        ref = gold.forward(want[-1], len(prompt) + g)
        want.append(og.argmax(ref))
    assert got.tolist() == want
    # a second call restarts the sequence at position 0 and must repeat itself
    assert eng.generate(prompt, 20).tolist() == want
    eng.close()


@pytest.mark.parametrize("path", ["fused", "graph"])
def test_engine_generate_across_chunk_boundary(gpu, og, path):
    """Greedy decoding across position 256, where the attention's cache of one head stops fitting
    one chunk and the chunk partials start going through the cross-block hand-off, inside one
    recorded step on the graph path.  The ids equal the CPU golden's, twice in a row."""
    cfg = dict(V=300, C=128, NL=2, NH=4, NKV=2, HD=32, FC=256, CTX=320)
    blob = gpu.qwen_random_blob(gpu.qwen_cfg(**cfg), seed=45, std=0.15)
    eng = gpu.QwenEngine(gpu.qwen_cfg(**cfg), blob, PATHS[path])
    prompt = [int(v) for v in np.random.default_rng(8).integers(0, cfg["V"], 248)]
    n = 16
    say(f"qwen generate across position 256, {path} path")
    got = eng.generate(prompt, n)
    gold = og.QwenGolden(og.qwen_cfg(**cfg), blob, NT)
    for p, t in enumerate(prompt):
        ref = gold.forward(t, p, p == len(prompt) - 1)
    want = [og.argmax(ref)]
    for g in range(n):
        ref = gold.forward(want[-1], len(prompt) + g)
        want.append(og.argmax(ref))
    assert got.tolist() == want
    assert eng.generate(prompt, n).tolist() == want
    eng.close()


def test_phase_times_leave_the_engine_usable(gpu):
    """sgpu_qwen_phase_times replays every decode phase (the argmax advancing the device position
    on each launch) and restores the position: afterwards greedy decoding still equals a fresh
    engine's, every phase time is positive, and a position outside the cache is refused."""
    cfg = gpu.qwen_cfg(**SMALL)
    blob = gpu.qwen_random_blob(cfg, seed=33, std=0.15)
    prompt = [int(v) for v in np.random.default_rng(5).integers(0, SMALL["V"], 9)]
    fresh = gpu.QwenEngine(cfg, blob, PATHS["graph"])
    want = fresh.generate(prompt, 20).tolist()
    fresh.close()
    eng = gpu.QwenEngine(cfg, blob, PATHS["graph"])
    for pos in (0, 7, SMALL["CTX"] - 1):
        t = eng.phase_times(pos, reps=3)
        say(f"phase times at {pos}: {t}")
        assert all(v > 0 and np.isfinite(v) for v in t.values()), t
    assert eng.generate(prompt, 20).tolist() == want
    us = np.zeros(len(gpu.QWEN_PHASES), np.float32)
    for bad in (-1, SMALL["CTX"]):
        assert gpu.lib().sgpu_qwen_phase_times(eng.h, bad, 3, us.ctypes.data) != 0
    eng.close()


def test_engine_full_generate_graph_token_identical(gpu, og):
    """Full Qwen2.5-0.5B architecture, graph path, on-device greedy loop: 32-token prompt,
    64 generated positions; the CPU golden, fed the same ids, picks the same argmax at every
    position."""
    cfg_g = gpu.qwen_default_cfg()
    blob = gpu.qwen_random_blob(cfg_g, seed=2024, std=0.02)
    eng = gpu.QwenEngine(cfg_g, blob, 2)
    prompt = [int(v) for v in np.random.default_rng(32).integers(0, cfg_g.V, 32)]
    got = eng.generate(prompt, 64).tolist()
    ocfg = og.qwen_cfg(cfg_g.V, cfg_g.C, cfg_g.NL, cfg_g.NH, cfg_g.NKV, cfg_g.HD, cfg_g.FC, cfg_g.CTX)
    gold = og.QwenGolden(ocfg, blob, NT)
    seq = prompt + got
    for p in range(len(prompt) + 64):
        ref = gold.forward(seq[p], p, p >= len(prompt) - 1)
        if p >= len(prompt) - 1:
            assert og.argmax(ref) == seq[p + 1], (p, og.argmax(ref), seq[p + 1])
    eng.close()


def test_engine_full_greedy_token_identical(gpu, og):
    """Random-init Qwen2.5-0.5B architecture (N(0, 0.02) weights), 32-token seeded prompt,
    64 greedy tokens on the reference launch sequence: every GPU token equals the CPU
    golden's argmax on the same history."""
    cfg_g = gpu.qwen_default_cfg()
    say("building full-size random weights")
    blob = gpu.qwen_random_blob(cfg_g, seed=2024, std=0.02)
    eng = gpu.QwenEngine(cfg_g, blob)
    ocfg = og.qwen_cfg(cfg_g.V, cfg_g.C, cfg_g.NL, cfg_g.NH, cfg_g.NKV, cfg_g.HD, cfg_g.FC, cfg_g.CTX)
    gold = og.QwenGolden(ocfg, blob, NT)
    ids = [int(v) for v in np.random.default_rng(32).integers(0, cfg_g.V, 32)]
    gaps, worst = [], 0.0
    tokens = list(ids)
    for p in range(32 + 64):
        want_logits = p >= len(ids) - 1
        got = eng.forward(tokens[p], p, want_logits)
        ref = gold.forward(tokens[p], p, want_logits)
        if not want_logits:
            continue
        g_tok, c_tok = int(np.argmax(got)), og.argmax(ref)
        top2 = np.sort(ref)[-2:]
        gaps.append(float(top2[1] - top2[0]))
        worst = max(worst, float(np.abs(got - ref).max() / np.abs(ref).max()))
        assert g_tok == c_tok, (p, g_tok, c_tok, gaps[-1])
        if len(tokens) < 32 + 64:
            tokens.append(g_tok)
        if p % 16 == 0:
            say(f"  pos {p}: token {g_tok} top-2 gap {gaps[-1]:.3e} worst rel err {worst:.2e}")
    assert len(tokens) == 96
    assert worst <= 1e-3
    say(f"greedy 64 tokens identical; min top-2 gap {min(gaps):.3e}, worst logit rel err {worst:.2e}")
    eng.close()


# ---- full-size parity that does not reduce to a few embeddings ----
# With the spec's N(0, 0.02) RMSNorm gains every layer's contribution is scaled by ~0.02, the
# residual stream is dominated by the current token's embedding, and greedy decoding falls
# into a 2-token cycle (18885, 77186, 32852, 77186, ...).  Two checks avoid that: the spec model
# teacher-forced over 64 seeded random ids (logits at every position), and a variant decoded
# free-running: RMSNorm gains 1 + N(0, 0.02) and the four projection matrices (qkv, o, gate|up,
# down) at twice the spec scale, so every layer mixes the history into the residual.
# Measured on this model and prompt (GPU reference path against the CPU golden, 64 greedy
# tokens): unit gains alone give 10 distinct tokens in 41 with long runs of one token;
# projections x2, 64 of 64 with the logits within 1.8e-5 of scale and every top-1/top-2 gap at
# least 16x the GPU/CPU difference.  Sharper variants amplify rounding differences through the
# 24 layers: qkv x6 gives 63 distinct tokens but logits 2.2e-2 of scale apart.

def full_cfgs(gpu, og):
    c = gpu.qwen_default_cfg()
    return c, og.qwen_cfg(c.V, c.C, c.NL, c.NH, c.NKV, c.HD, c.FC, c.CTX)


def rich_variant(blob, c, seed=7, proj_scale=2.0):
    """Every RMSNorm gain of the flat file set to fp16(1 + N(0, 0.02)), seeded, and the qkv, o,
    gate|up and down weights multiplied by proj_scale (re-rounded to fp16): offsets of the
    qwen_engine.c:61-75 layout -- embedding, RoPE tables, then per layer in_ln, qkv W, qkv b,
    o W, post_ln, gate|up W, down W, then the final norm."""
    h = blob.view(np.uint16)
    qkv = c.C + 2 * c.NKV * c.HD
    base = (c.V * c.C * 2 + 2 * c.CTX * (c.HD // 2) * 4) // 2
    lstride = c.C + qkv * c.C + qkv + c.C * c.C + c.C + 2 * c.FC * c.C + c.C * c.FC
    rng = np.random.default_rng(seed)
    gain = lambda: (1.0 + 0.02 * rng.standard_normal(c.C)).astype(np.float16).view(np.uint16)

    def scale(a, n):
        w = h[a:a + n]
        w[:] = (w.view(np.float16).astype(np.float32) * proj_scale).astype(np.float16).view(np.uint16)

    for l in range(c.NL):
        p = base + l * lstride
        h[p:p + c.C] = gain()                          # input RMSNorm
        p += c.C
        scale(p, qkv * c.C)                            # qkv W
        p += qkv * c.C + qkv
        scale(p, c.C * c.C)                            # o W
        p += c.C * c.C
        h[p:p + c.C] = gain()                          # post-attention RMSNorm
        p += c.C
        scale(p, 2 * c.FC * c.C)                       # gate|up W
        p += 2 * c.FC * c.C
        scale(p, c.C * c.FC)                           # down W
    e = base + c.NL * lstride
    h[e:e + c.C] = gain()                              # final RMSNorm
    return blob


def check_position(p, got, ref, gaps, stats):
    """Logits within 1e-3 of the logit scale; the argmax equal unless the reference's margin of
    its top token over the GPU's pick is within 4x this position's RMS logit error (a near-tie,
    counted and printed).  The RMS, not the largest error, sets the bar: a flip is always
    within twice the largest error of the two logits involved, so only an outlier error on
    exactly those two logits can flip a wider margin, and that fails the test."""
    err = np.abs(got.astype(np.float64) - ref)
    stats["worst"] = max(stats["worst"], float(err.max() / np.abs(ref).max()))
    assert err.max() <= 1e-3 * np.abs(ref).max(), (p, float(err.max()), float(np.abs(ref).max()))
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
    """The spec model (seed 2024, N(0, 0.02)) and the CPU golden's logits for 64 seeded random
    ids fed one position at a time."""
    c, oc = full_cfgs(gpu, og)
    say("full spec model: building weights and 64 golden positions")
    blob = gpu.qwen_random_blob(c, seed=2024, std=0.02)
    ids = [int(v) for v in np.random.default_rng(64).integers(0, c.V, 64)]
    gold = og.QwenGolden(oc, blob, NT)
    logits = np.stack([gold.forward(t, p) for p, t in enumerate(ids)])
    return c, blob, ids, logits


@pytest.mark.parametrize("path", ["reference", "graph"])
def test_engine_full_teacher_forced(gpu, full_spec, path):
    """Full Qwen2.5-0.5B architecture (spec init), 64 random ids teacher-forced: the logits of
    every position against the CPU golden (1e-3 of scale, argmax equal), on the reference
    launch sequence and on the replayed graph."""
    c, blob, ids, logits = full_spec
    eng = gpu.QwenEngine(c, blob, PATHS[path])
    gaps, stats = [], {"worst": 0.0, "ties": 0}
    for p, t in enumerate(ids):
        check_position(p, eng.forward(t, p, True).copy(), logits[p], gaps, stats)
    eng.close()
    say(f"{path}: 64 teacher-forced positions, worst logit error {stats['worst']:.2e} of scale, "
        f"min top-1/top-2 gap {min(gaps):.3e}, median {np.median(gaps):.3e}, near-ties {stats['ties']} {stats.get('flips', [])}")
    assert stats["ties"] <= 2


@pytest.fixture(scope="module")
def full_variant(gpu, og):
    """The rich variant (unit RMSNorm gains, projections x2), 32-id prompt, and the CPU golden's own
    greedy continuation of 64 tokens with the logits it took each one from."""
    c, oc = full_cfgs(gpu, og)
    say("full variant model: building weights and the golden's greedy run")
    blob = rich_variant(gpu.qwen_random_blob(c, seed=2024, std=0.02), c)
    prompt = [int(v) for v in np.random.default_rng(32).integers(0, c.V, 32)]
    gold = og.QwenGolden(oc, blob, NT)
    seq, logits = list(prompt), []
    for p in range(32 + 64):
        ref = gold.forward(seq[p], p, p >= 31)
        if p >= 31:
            logits.append(ref)
            if len(seq) < 32 + 64 + 1:
                seq.append(og.argmax(ref))
    return c, blob, prompt, seq[32:], np.stack(logits)


@pytest.mark.parametrize("path", ["reference", "graph"])
def test_engine_full_variant_greedy(gpu, full_variant, path):
    """Free-running greedy decode on the rich variant: 64 tokens token-identical to the CPU
    golden's own greedy run, which does not cycle (at least 24 distinct tokens of 64).  The
    reference path runs the host loop of the reference (logits to the host, argmax there,
    each position's logits checked); the graph path runs sgpu_qwen_generate's on-device loop."""
    c, blob, prompt, want, logits = full_variant
    distinct = len(set(want[:64]))
    say(f"golden greedy continuation: {want[:12]} ..., {distinct} distinct of 64")
    assert distinct >= 24
    eng = gpu.QwenEngine(c, blob, PATHS[path])
    if path == "graph":
        got = eng.generate(prompt, 64).tolist()
        assert got == want[:65], next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)
    else:
        gaps, stats = [], {"worst": 0.0, "ties": 0}
        seq = list(prompt)
        for p in range(32 + 64):
            out = eng.forward(seq[p], p, p >= 31)
            if p >= 31:
                tok = check_position(p, out.copy(), logits[p - 31], gaps, stats)
                assert tok == want[p - 31], (p, tok, want[p - 31])
                seq.append(tok)
        say(f"reference path: 64 greedy tokens identical, worst logit error {stats['worst']:.2e}, "
            f"min top-1/top-2 gap {min(gaps):.3e}")
    eng.close()


def test_engine_cli_json(gpu):
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "qwen_engine")
    runs = {}
    for path, extra in (("reference", []), ("graph", []), ("graph", ["--batch-prefill"])):
        out = subprocess.run([exe, "--random", "7", "--prompt-random", "8", "--gen", "6", "--json", "--path", path]
                             + extra, capture_output=True, text=True, timeout=300)
        assert out.returncode == 0, out.stderr
        d = json.loads(out.stdout.strip().splitlines()[-1])
        assert d["done"] and d["tok_s"] > 0
        runs[path + "".join(extra)] = d["ids"]
    assert runs["reference"] == runs["graph"] == runs["graph--batch-prefill"]


def test_engine_serve_protocol(gpu):
    """--serve (qwen_engine.c:406-444): per request u32 T, T u32 ids, u32 max_gen on stdin;
    u32 M then M u32 ids (the prompt echoed, then the greedy continuation) on stdout.  Two
    requests on one process; each continuation equals sgpu_qwen_generate on the same weights
    (the CLI's --random SEED model) up to an EOT / <|im_end|> stop."""
    import struct

    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "qwen_engine")
    reqs = [([5, 17, 9000, 151000, 42], 6), ([123] * 3 + [7], 4)]
    payload = b"".join(struct.pack(f"<I{len(ids)}II", len(ids), *ids, g) for ids, g in reqs)
    answers = []
    for extra in ([], ["--batch-prefill"]):
        out = subprocess.run([exe, "--random", "7", "--serve"] + extra, input=payload, capture_output=True,
                             timeout=300)
        assert out.returncode == 0, out.stderr.decode()
        buf, off, got = out.stdout, 0, []
        for _ in reqs:
            (m,) = struct.unpack_from("<I", buf, off)
            got.append(list(struct.unpack_from(f"<{m}I", buf, off + 4)))
            off += 4 + 4 * m
        assert off == len(buf)
        answers.append(got)
    assert answers[0] == answers[1]
    cfg = gpu.qwen_default_cfg()
    eng = gpu.QwenEngine(cfg, gpu.qwen_random_blob(cfg, seed=7, std=0.02), 2)
    for (ids, g), resp in zip(reqs, got):
        assert resp[:len(ids)] == ids
        want = eng.generate(ids, g).tolist()
        cont = resp[len(ids):]
        stop = next((i for i, t in enumerate(want) if t in (151643, 151645)), None)
        assert cont == (want if stop is None else want[:stop + 1]), (cont, want)
    eng.close()


# ---- the CLI's own self-test (--selftest / --debug, qwen_engine.c:446-521) ----
TRACE_RE = r"trace p0 L(\d+): max\|d\|=([0-9.]+) \(\|gpu\|~([0-9.]+)\)"


def check_selftest_output(text, NL):
    import re

    traces = re.findall(TRACE_RE, text)
    assert [int(t[0]) for t in traces] == list(range(NL)), text[-2000:]
    for layer, d, g in traces:
        assert float(d) <= 1e-3 * max(float(g), 1.0), (layer, d, g)
    assert "SELFTEST: PASS" in text and "argmax" in text and "MATCH" in text, text[-2000:]
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


@pytest.mark.parametrize("path", ["reference", "graph"])
def test_cli_selftest(gpu, path, tmp_path):
    """bin/qwen_engine --selftest 3 on the full random-init model: the per-layer residual trace at
    position 0 and the logits at position 2 against the program's own serial CPU forward, then
    priming continues from position 3 and generation runs to the end."""
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "qwen_engine")
    say(f"qwen_engine --selftest 3 --path {path}")
    out = subprocess.run([exe, "--random", "2024", "--selftest", "3", "--gen", "4", "--path", path],
                         capture_output=True, text=True, timeout=600, cwd=tmp_path)
    assert out.returncode == 0, out.stderr[-2000:]
    check_selftest_output(out.stdout, 24)
    assert "positions 0..2 by the self-test" in out.stdout and "ENGINE_DONE" in out.stdout
    assert not (tmp_path / "trace_g.bin").exists()


def test_cli_selftest_debug(gpu, tmp_path):
    """--debug adds the layer-0 stage lines, the GPU's (g.*, the reference launch sequence)
    before the CPU forward's (c.*), agreeing where both print a stage, and writes both layer
    traces."""
    exe = os.path.join(ROOT, "switch-l4t-gpu_amd", "bin", "qwen_engine")
    say("qwen_engine --selftest 1 --debug")
    out = subprocess.run([exe, "--random", "7", "--selftest", "1", "--debug", "--gen", "1"],
                         capture_output=True, text=True, timeout=600, cwd=tmp_path)
    assert out.returncode == 0, out.stderr[-2000:]
    check_selftest_output(out.stdout, 24)
    for tag in ("embed", "ln1", "qkv", "ao", "res1"):
        assert f"c.{tag}" in out.stdout
    st = stage_lines(out.stdout)
    assert all(("g", t) in st for t in ("ln1", "qkv", "scores", "probs", "attnout", "res1", "gate", "swiglu", "res2")), sorted(st)
    assert out.stdout.index("g.ln1") < out.stdout.index("c.ln1")
    check_stages_agree(st, ("ln1", "qkv", "res1"), 1e-3)
    g = np.fromfile(tmp_path / "trace_g.bin", np.float32)
    c = np.fromfile(tmp_path / "trace_c.bin", np.float32)
    assert g.size == c.size == 24 * 896
    assert np.abs(g - c).max() <= 1e-3 * max(np.abs(g).max(), 1.0)


def test_forward_stages(gpu):
    """sgpu_qwen_forward_stages: the reference's nine layer-0 stages in launch order, the last
    one bit-identical to the layer trace of the same launch sequence; at position 0 every
    head's softmax is exactly 1 and its output is its KV group's v."""
    c = gpu.qwen_cfg(**SMALL)
    blob = gpu.qwen_random_blob(c, seed=11, std=0.15)
    eng = gpu.QwenEngine(c, blob, PATHS["graph"])
    logits_s, st = eng.forward_stages(5, 0)
    logits_s = logits_s.copy()
    names = [t for t, _ in st]
    assert names == ["ln1", "qkv", "scores", "probs", "attnout", "res1", "gate", "swiglu", "res2"]
    v = dict(st)
    C, NH, NKV, HD, FC = SMALL["C"], SMALL["NH"], SMALL["NKV"], SMALL["HD"], SMALL["FC"]
    assert [len(v[k]) for k in names] == [C, C + 2 * NKV * HD, NH, NH, C, C, FC, FC, C]
    assert np.array_equal(v["probs"], np.ones(NH, np.float32))
    vpart = v["qkv"][C + NKV * HD:]
    want = np.concatenate([vpart[(h // (NH // NKV)) * HD:(h // (NH // NKV) + 1) * HD] for h in range(NH)])
    assert np.array_equal(v["attnout"], want)
    logits_t, trace = eng.forward_trace(5, 0)
    assert np.array_equal(v["res2"], trace[0]) and np.array_equal(logits_s, logits_t)
    eng.close()


def test_forward_trace_is_the_reference_forward(gpu):
    """sgpu_qwen_forward_trace computes what the reference path computes, bit for bit, on an
    engine of any path, and its last layer's trace is the residual the logits come from."""
    c = gpu.qwen_cfg(V=512, C=128, NL=3, NH=4, NKV=2, HD=32, FC=256, CTX=64)
    blob = gpu.qwen_random_blob(c, seed=11, std=0.15)
    ref = gpu.QwenEngine(c, blob, gpu.QWEN_PATH_REFERENCE)
    tr_eng = gpu.QwenEngine(c, blob, gpu.QWEN_PATH_GRAPH)
    ids = [5, 77, 301, 2, 9]
    for p, t in enumerate(ids):
        want = ref.forward(t, p).copy()
        got, trace = tr_eng.forward_trace(t, p)
        assert np.array_equal(got, want), p
        assert trace.shape == (3, 128) and np.all(np.isfinite(trace))
    ref.close()
    tr_eng.close()
