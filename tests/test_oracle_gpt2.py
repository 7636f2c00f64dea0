"""Pins the GPT-2 decode oracle (og_gpt2_forward, restating gpt2_engine.c:363-420 with cpu_ln
:333-341) against the GPT-2 model of the transformers library on the same weights: the
flat fp32 file (gpt2_engine.c:50-70) is loaded into GPT2LMHeadModel (Conv1D weights are
the transposes of the engine's [out, in] rows, conv_gpt2.py:35-47), and the logits of every
position of a sequence must match the oracle's sequential KV-cache decode.  CPU only."""
import numpy as np
import pytest

SMALL = dict(V=1000, C=768, NL=2, NH=12, HD=64, FC=3072, CTX=64)


def split(w, cfg):
    V, C, NL, FC, CTX = cfg["V"], cfg["C"], cfg["NL"], cfg["FC"], cfg["CTX"]
    wte = w[:V * C].reshape(V, C)
    wpe = w[V * C:V * C + CTX * C].reshape(CTX, C)
    base = V * C + CTX * C
    lf = 2 * C + 3 * C * C + 3 * C + C * C + C + 2 * C + FC * C + FC + FC * C + C
    layers = []
    for l in range(NL):
        p = base + l * lf
        take = lambda n, shape=None: (w[p:p + n].reshape(shape) if shape else w[p:p + n])
        L = {}
        for name, n, shape in [("ln1w", C, None), ("ln1b", C, None), ("qkvw", 3 * C * C, (3 * C, C)),
                               ("qkvb", 3 * C, None), ("aow", C * C, (C, C)), ("aob", C, None),
                               ("ln2w", C, None), ("ln2b", C, None), ("fcw", FC * C, (FC, C)), ("fcb", FC, None),
                               ("projw", C * FC, (C, FC)), ("projb", C, None)]:
            L[name] = take(n, shape)
            p += n
        layers.append(L)
    end = base + NL * lf
    return wte, wpe, layers, w[end:end + C], w[end + C:end + 2 * C]


def hf_logits(w, cfg, ids):
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    hc = transformers.GPT2Config(vocab_size=cfg["V"], n_positions=cfg["CTX"], n_embd=cfg["C"], n_layer=cfg["NL"],
                                 n_head=cfg["NH"], n_inner=cfg["FC"], activation_function="gelu_new",
                                 layer_norm_epsilon=1e-5, resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0,
                                 attn_implementation="eager")
    model = transformers.GPT2LMHeadModel(hc).float().eval()
    wte, wpe, layers, lnfw, lnfb = split(w, cfg)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32))
    with torch.no_grad():
        tr = model.transformer
        tr.wte.weight.copy_(T(wte))
        tr.wpe.weight.copy_(T(wpe))
        for l, L in enumerate(layers):
            h = tr.h[l]
            h.ln_1.weight.copy_(T(L["ln1w"])); h.ln_1.bias.copy_(T(L["ln1b"]))
            h.attn.c_attn.weight.copy_(T(L["qkvw"].T)); h.attn.c_attn.bias.copy_(T(L["qkvb"]))
            h.attn.c_proj.weight.copy_(T(L["aow"].T)); h.attn.c_proj.bias.copy_(T(L["aob"]))
            h.ln_2.weight.copy_(T(L["ln2w"])); h.ln_2.bias.copy_(T(L["ln2b"]))
            h.mlp.c_fc.weight.copy_(T(L["fcw"].T)); h.mlp.c_fc.bias.copy_(T(L["fcb"]))
            h.mlp.c_proj.weight.copy_(T(L["projw"].T)); h.mlp.c_proj.bias.copy_(T(L["projb"]))
        tr.ln_f.weight.copy_(T(lnfw)); tr.ln_f.bias.copy_(T(lnfb))
        model.lm_head.weight = tr.wte.weight
        return model(torch.tensor([ids]), use_cache=False).logits[0].numpy()


def weights(sg, cfg, seed, unit_gains):
    w = sg.gpt2_random_weights(sg.gpt2_cfg(**cfg), seed, 0.03)
    if unit_gains:   # LayerNorm gains near 1 so the nonlinear parts carry real signal
        wte, wpe, layers, lnfw, _ = split(w, cfg)
        for L in layers:
            L["ln1w"] += 1.0
            L["ln2w"] += 1.0
            L["fcb"] *= 30.0
        lnfw += 1.0
    return w


@pytest.mark.parametrize("unit_gains", [False, True])
def test_gpt2_forward_matches_transformers(og, sg, unit_gains):
    cfg = SMALL
    w = weights(sg, cfg, 17, unit_gains)
    assert w.size == og.gpt2_file_floats(og.gpt2_cfg(**cfg))
    ids = [int(v) for v in np.random.default_rng(9).integers(0, cfg["V"], 12)]
    g = og.Gpt2Golden(og.gpt2_cfg(**cfg), w)
    got = np.stack([g.forward(t, p) for p, t in enumerate(ids)])
    want = hf_logits(w, cfg, ids)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 2e-5 * scale + 1e-7, (np.abs(got - want).max(), scale)
    assert [int(np.argmax(r)) for r in got] == [int(np.argmax(r)) for r in want]


def test_gpt2_file_floats(og, sg):
    """124,439,808 floats at the GPT-2 124M dims (conv_gpt2.py:67, make_random_bin.py:6)."""
    import ctypes

    assert og.gpt2_file_floats(og.gpt2_cfg()) == 124_439_808
    assert sg.lib().sgpu_gpt2_file_floats(ctypes.byref(sg.gpt2_cfg())) == 124_439_808


def test_layernorm_matches_torch(og):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(768) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(768).astype(np.float32)
    b = rng.standard_normal(768).astype(np.float32)
    got = og.layernorm(x, w, b, 1e-5)
    want = torch.nn.functional.layer_norm(torch.from_numpy(x).double(), (768,), torch.from_numpy(w).double(),
                                          torch.from_numpy(b).double(), eps=1e-5).numpy()
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)


def test_gpt2_threads_bitwise(og, sg):
    cfg = SMALL
    w = weights(sg, cfg, 3, True)
    a, b = og.Gpt2Golden(og.gpt2_cfg(**cfg), w, 1), og.Gpt2Golden(og.gpt2_cfg(**cfg), w, 4)
    for p, t in enumerate([5, 999, 0, 5]):
        assert np.array_equal(a.forward(t, p), b.forward(t, p))
