"""Pins the decode oracle (og_qwen_forward, restating qwen_engine.c:292-358) against the
Qwen2 model of the transformers library: the same random-init weights, decoded with the
reference h2f, loaded into transformers' Qwen2ForCausalLM (fp32, eager attention), must give
the same logits at every position as the oracle's sequential KV-cache decode.  This fixes
the layout offsets, the q|k|v and gate|up row splits, the half-split RoPE convention, GQA
head grouping, the softmax/mix order and the tied lm_head independently of the restatement.
CPU only."""
import numpy as np
import pytest

SMALL = dict(V=512, C=128, NL=2, NH=4, NKV=2, HD=32, FC=256, CTX=64)


def split_blob(og, blob, cfg):
    """Slice the flat weight file (qwen_engine.c:61-75) into decoded fp32 tensors."""
    V, C, NL, NH, NKV, HD, FC, CTX = (cfg[k] for k in ("V", "C", "NL", "NH", "NKV", "HD", "FC", "CTX"))
    KV, QKV = NKV * HD, C + 2 * NKV * HD
    h = blob.view(np.uint16)
    dec = lambda a: og.h2f_array(a)
    off = 0
    emb = dec(h[off:off + V * C]).reshape(V, C)
    off = (V * C * 2 + 2 * CTX * (HD // 2) * 4) // 2
    lstride = C + QKV * C + QKV + C * C + C + 2 * FC * C + C * FC
    layers = []
    for l in range(NL):
        b = off + l * lstride
        p = b
        ln1 = dec(h[p:p + C]); p += C
        qkvw = dec(h[p:p + QKV * C]).reshape(QKV, C); p += QKV * C
        qkvb = dec(h[p:p + QKV]); p += QKV
        ow = dec(h[p:p + C * C]).reshape(C, C); p += C * C
        ln2 = dec(h[p:p + C]); p += C
        gu = dec(h[p:p + 2 * FC * C]).reshape(2 * FC, C); p += 2 * FC * C
        down = dec(h[p:p + C * FC]).reshape(C, FC); p += C * FC
        layers.append(dict(ln1=ln1, qkvw=qkvw, qkvb=qkvb, ow=ow, ln2=ln2, gu=gu, down=down))
    lnf = dec(h[off + NL * lstride: off + NL * lstride + C])
    return emb, layers, lnf, KV


def hf_logits(og, blob, cfg, ids):
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    C, FC = cfg["C"], cfg["FC"]
    hc = transformers.Qwen2Config(vocab_size=cfg["V"], hidden_size=C, intermediate_size=FC,
                                  num_hidden_layers=cfg["NL"], num_attention_heads=cfg["NH"],
                                  num_key_value_heads=cfg["NKV"], max_position_embeddings=cfg["CTX"],
                                  rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=True,
                                  hidden_act="silu", attn_implementation="eager")
    model = transformers.Qwen2ForCausalLM(hc).float().eval()
    emb, layers, lnf, KV = split_blob(og, blob, cfg)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32))
    with torch.no_grad():
        m = model.model
        m.embed_tokens.weight.copy_(T(emb))
        for l, L in enumerate(layers):
            lay = m.layers[l]
            a = lay.self_attn
            a.q_proj.weight.copy_(T(L["qkvw"][:C])); a.q_proj.bias.copy_(T(L["qkvb"][:C]))
            a.k_proj.weight.copy_(T(L["qkvw"][C:C + KV])); a.k_proj.bias.copy_(T(L["qkvb"][C:C + KV]))
            a.v_proj.weight.copy_(T(L["qkvw"][C + KV:])); a.v_proj.bias.copy_(T(L["qkvb"][C + KV:]))
            a.o_proj.weight.copy_(T(L["ow"]))
            lay.input_layernorm.weight.copy_(T(L["ln1"]))
            lay.post_attention_layernorm.weight.copy_(T(L["ln2"]))
            lay.mlp.gate_proj.weight.copy_(T(L["gu"][:FC]))
            lay.mlp.up_proj.weight.copy_(T(L["gu"][FC:]))
            lay.mlp.down_proj.weight.copy_(T(L["down"]))
        m.norm.weight.copy_(T(lnf))
        model.lm_head.weight = m.embed_tokens.weight
        out = model(torch.tensor([ids]), use_cache=False).logits[0]
    return out.numpy()


def oracle_logits(og, blob, cfg, ids, nthreads=1):
    c = og.qwen_cfg(**cfg)
    g = og.QwenGolden(c, blob, nthreads)
    return np.stack([g.forward(t, p, True) for p, t in enumerate(ids)])


@pytest.mark.parametrize("std", [0.02, 0.15])
def test_qwen_forward_matches_transformers(og, sg, std):
    cfg = SMALL
    blob = sg.qwen_random_blob(sg.qwen_cfg(**cfg), seed=11, std=std)
    assert blob.nbytes == og.qwen_file_bytes(og.qwen_cfg(**cfg))
    ids = [int(v) for v in np.random.default_rng(3).integers(0, cfg["V"], 14)]
    got = oracle_logits(og, blob, cfg, ids)
    want = hf_logits(og, blob, cfg, ids)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 2e-5 * scale + 1e-7, (np.abs(got - want).max(), scale)
    assert [int(np.argmax(r)) for r in got] == [int(np.argmax(r)) for r in want]


def test_qwen_forward_threads_bitwise_and_cache(og, sg):
    cfg = SMALL
    blob = sg.qwen_random_blob(sg.qwen_cfg(**cfg), seed=5, std=0.1)
    ids = [7, 300, 5, 5, 511]
    a = oracle_logits(og, blob, cfg, ids, nthreads=1)
    b = oracle_logits(og, blob, cfg, ids, nthreads=4)
    assert np.array_equal(a, b)
    # position 0 only attends to itself: its logits do not depend on any other token
    c = oracle_logits(og, blob, cfg, [7])
    assert np.array_equal(a[0], c[0])


def test_full_file_size(og, sg):
    """FILE_BYTES at the Qwen2.5-0.5B dims and CTX 8192 (qwen_engine.c:61-67)."""
    full = dict(V=151936, C=896, NL=24, NH=14, NKV=2, HD=64, FC=4864, CTX=8192)
    import ctypes

    assert og.qwen_file_bytes(og.qwen_cfg(**full)) == 990_162_688
    assert sg.lib().sgpu_qwen_file_bytes(ctypes.byref(sg.qwen_cfg(**full))) == 990_162_688


def test_oracle_rejects_bad_position(og, sg):
    cfg = SMALL
    blob = sg.qwen_random_blob(sg.qwen_cfg(**cfg), seed=1)
    g = og.QwenGolden(og.qwen_cfg(**cfg), blob)
    with pytest.raises(ValueError):
        g.forward(0, cfg["CTX"])
    with pytest.raises(ValueError):
        g.forward(cfg["V"], 0)
