"""Gemma 4 on the host (no GPU): the gemma4 GGUF files of llama.cpp's converter
and their refusals (TTestInferQwen3.Gemma4Gguf*, tests/test.infer.qwen3.pas:
4795-4830), the CPU oracle decoding them against the float32 logits
transformers wrote for the same weights (tiny-gemma4: sliding and full layers
of their own heads, K=V, two rotary sets, the dense block beside 8 experts,
layer scalars, the softcap; tiny-gemma4/dense), and closed forms of GeGLU, the
softcap and the second rotary set (backend.cpu.pas:1836-1860, decoder.pas:
1293-1312, :1742-1752)."""
import os

import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O

GG = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gguf")
EXP = np.load(os.path.join(GG, "expected.npz"))


def cases(tag):
    out, k = [], 0
    while f"{tag}/case{k}.ids" in EXP.files:
        out.append({f: EXP[f"{tag}/case{k}.{f}"] for f in ("ids", "logits", "greedy")})
        k += 1
    return out


def cos(a, b):
    a, b = a.ravel().astype(np.float64), b.ravel().astype(np.float64)
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


@pytest.mark.parametrize("name,why", [
    ("bad-arch.gguf", "architecture"), ("bad-ple.gguf", "per-layer embeddings"),
    ("bad-shared.gguf", "shared KV layers"), ("bad-ffn.gguf", "width per layer"),
    ("bad-scaling.gguf", "rope scaling"), ("bad-rope.gguf", "rotating 8"),
    ("bad-pattern.gguf", "sliding_window_pattern"), ("bad-freqs.gguf", r"rope_freqs.weight\[2\]"),
    ("bad-head.gguf", "untied head"), ("bad-missing.gguf", "blk.1.ffn_down_exps.scale"),
    ("bad-extra.gguf", "understood"), ("bad-swa-v.gguf", "blk.2.attn_v.weight")])
def test_gemma4_damaged_files_refused(name, why):
    # the reasons of the reference's own checks (test.infer.qwen3.pas:4807-4818)
    with pytest.raises(H.FormatError, match=why):
        H.GgufSpec(os.path.join(GG, "bad", "gemma4", name))


def test_gemma4_settings_of_the_files():
    s = H.GgufSpec(os.path.join(GG, "gemma4", "q8_0.gguf")).struct
    assert (s.layers, s.head_dim, s.kv_heads, s.rope2_pairs) == (4, 16, 2, 4)
    assert [s.layer[i].window for i in range(4)] == [5, 0, 5, 0]
    assert [s.layer[i].head_dim for i in range(4)] == [0, 32, 0, 32]
    assert [s.layer[i].kv_heads for i in range(4)] == [2, 1, 2, 1]
    assert [s.layer[i].k_is_v for i in range(4)] == [0, 1, 0, 1]
    assert [s.layer[i].moe for i in range(4)] == [H.FFN_DENSE_MOE] * 4
    assert (s.activation, s.value_norm, s.attention_scale, s.logit_softcap) == (H.ACT_GELU_TANH, 1, 1.0, 3.0)
    assert s.embed_scale == np.float32(8.0) and s.rope_theta == 10000.0 and s.rope2_theta == 1e6
    d = H.GgufSpec(os.path.join(GG, "gemma4", "dense-q8_0.gguf")).struct
    assert [d.layer[i].window for i in range(6)] == [5] * 5 + [0]
    assert [d.layer[i].kv_heads for i in range(6)] == [2] * 6
    assert [d.layer[i].k_is_v for i in range(6)] == [0] * 6
    assert [d.layer[i].moe for i in range(6)] == [H.FFN_DENSE] * 6
    # 15 pairs of a head of 44 (2 * 15 / 44 * 44 is 29.999... in double)
    r = H.GgufSpec(os.path.join(GG, "gemma4", "rope44.gguf")).struct
    assert r.rope2_pairs == 15 and r.layer[1].head_dim == 44


@pytest.mark.parametrize("file,tag", [("bf16", "gemma4"), ("dense-bf16", "gemma4-dense")])
def test_oracle_gemma4_bf16_vs_transformers(file, tag):
    # BF16 widened exactly: transformers' float32 (soft-capped) logits within
    # 2e-5, in one pass and one token at a time, both Linear arithmetics, and
    # its greedy tokens
    s = H.GgufSpec(os.path.join(GG, "gemma4", file + ".gguf"))
    for c in cases(tag):
        for f32 in (False, True):
            lg = O.Model(s, 128, f32=f32).forward(c["ids"], all_logits=True)
            assert np.abs(lg - c["logits"]).max() < 2e-5
        m = O.Model(s, 128)
        st = np.stack([m.forward(c["ids"][i:i + 1]) for i in range(len(c["ids"]))])
        assert np.abs(st - c["logits"]).max() < 2e-5
        ids, _ = O.Model(s, 128).greedy(c["ids"], len(c["greedy"]))
        assert np.array_equal(ids, c["greedy"])


@pytest.mark.parametrize("file,tag", [("q8_0", "gemma4"), ("dense-q8_0", "gemma4-dense")])
def test_oracle_gemma4_q8_0_vs_transformers(file, tag):
    # Q8_0 matrices (the experts and the embedding too) against the float32
    # logits of the BF16 weights: within the Q8_0 error of a chaotic tiny model
    s = H.GgufSpec(os.path.join(GG, "gemma4", file + ".gguf"))
    for c in cases(tag):
        for f32 in (False, True):
            lg = O.Model(s, 128, f32=f32).forward(c["ids"], all_logits=True)
            assert np.abs(lg - c["logits"]).max() < 1.0
            assert cos(lg, c["logits"]) > 0.98


# ------------------------------------------------------------ closed forms
def test_geglu_closed_form():
    g = np.array([-30.0, -3.0, -0.5, 0.0, 0.7, 2.0, 12.0, 40.0], np.float32)
    u = np.linspace(-2, 2, g.size).astype(np.float32)
    gd = g.astype(np.float64)
    want = 0.5 * gd * (1 + np.tanh(np.sqrt(2 / np.pi) * (gd + 0.044715 * gd ** 3))) * u
    assert np.allclose(O.geglu(g, u), want, rtol=3e-7, atol=1e-30)


def test_softcap_closed_form():
    x = np.array([-500.0, -9.0, -1.0, 0.0, 0.25, 3.0, 61.0, 500.0], np.float32)
    want = np.tanh(x.astype(np.float64) / 3.0) * 3.0
    assert np.allclose(O.softcap(x, 3.0), want, rtol=3e-7, atol=1e-7)


def test_rotary2_closed_form():
    # 1 / theta2 ^ (2i / hd2) for the rotating pairs, frequency 0 after them
    s = H.GgufSpec(os.path.join(GG, "gemma4", "rope44.gguf"))
    c, sn = O.rotary2(s, 44, 7, 3)
    i = np.arange(22)
    f = np.where(i < 15, 1.0 / 1e6 ** (2 * i / 44.0), 0.0)
    ang = (7 + np.arange(3))[:, None] * f[None, :]
    assert np.allclose(c, np.cos(ang), rtol=1e-6, atol=1e-6)
    assert np.allclose(sn, np.sin(ang), rtol=1e-6, atol=1e-6)
    assert np.all(c[:, 15:] == 1) and np.all(sn[:, 15:] == 0)
