"""Qwen3.5 on the host (no GPU): the qwen35 GGUF files of llama.cpp's converter
and their refusals (TTestInferQwen35, tests/test.infer.qwen35.pas:1040-1140),
the CPU oracle decoding them against the float32 logits transformers wrote for
the same weights (tiny-qwen35 and tiny-qwen35/text, tests/golden/gguf/
expected.npz: one pass, one token at a time, greedy), and closed forms of the
DeltaNet steps (DeltaPrep decoder.pas:2755-2855, DeltaRule backend.cpu.pas:
1890-1972, GateBySigmoid decoder.pas:2594-2610)."""
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
        out.append({f: EXP[f"{tag}/case{k}.{f}"] for f in ("ids", "logits", "logits_steps", "greedy")})
        k += 1
    return out


def cos(a, b):
    a, b = a.ravel().astype(np.float64), b.ravel().astype(np.float64)
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


@pytest.mark.parametrize("name,why", [
    ("bad-arch.gguf", "qwen3next"), ("bad-prism.gguf", "transformed basis"),
    ("bad-inner.gguf", "inner size"), ("bad-mtp.gguf", "prediction layers"),
    ("bad-recurrent.gguf", "recurrent_layers"), ("bad-rope.gguf", "rotating values"),
    ("bad-scaling.gguf", "rope scaling"), ("bad-missing.gguf", "blk.1.ssm_a"),
    ("bad-extra.gguf", "understood"), ("bad-ssm-a.gguf", "no -exp(A_log)")])
def test_qwen35_damaged_files_refused(name, why):
    with pytest.raises(H.FormatError, match=why.replace("(", r"\(").replace(")", r"\)")):
        H.GgufSpec(os.path.join(GG, "bad", "qwen35", name))


def test_qwen35_settings_of_the_files():
    # tiny-qwen35: 4 layers (the mtp block after them left out), every 4th
    # full, a quarter of each head rotating; text: recurrent_layers, 2 key
    # heads read by 4 value heads in the tiled order, a convolution of 3
    s = H.GgufSpec(os.path.join(GG, "qwen35", "q8_0.gguf")).struct
    assert (s.layers, s.rope_dims, s.head_dim, s.lin_conv, s.lin_tiled) == (4, 8, 32, 4, 0)
    assert [s.layer[i].mixer for i in range(4)] == [1, 1, 1, 0]
    assert [s.layer[i].output_gate for i in range(4)] == [0, 0, 0, 1]
    assert (s.lin_key_heads, s.lin_value_heads, s.lin_key_dim, s.lin_value_dim) == (2, 2, 16, 16)
    t = H.GgufSpec(os.path.join(GG, "qwen35", "text-q8_0.gguf")).struct
    assert (t.layers, t.rope_dims, t.lin_conv, t.lin_tiled) == (5, 16, 3, 1)
    assert [t.layer[i].mixer for i in range(5)] == [1, 0, 1, 1, 0]
    assert (t.lin_key_heads, t.lin_value_heads, t.lin_key_dim, t.lin_value_dim) == (2, 4, 16, 8)
    assert t.head.data  # untied


@pytest.mark.parametrize("file,tag", [("bf16", "qwen35"), ("text-bf16", "qwen35-text")])
def test_oracle_qwen35_bf16_vs_transformers(file, tag):
    # BF16 matrices widen exactly: transformers' float32 logits within 1e-5,
    # in one pass (the chunked rule) and one token at a time (the recurrent
    # rule), in both Linear arithmetics, and its greedy tokens
    s = H.GgufSpec(os.path.join(GG, "qwen35", file + ".gguf"))
    for c in cases(tag):
        for f32 in (False, True):
            lg = O.Model(s, 128, f32=f32).forward(c["ids"], all_logits=True)
            assert np.abs(lg - c["logits"]).max() < 1e-5
        m = O.Model(s, 128)
        st = np.stack([m.forward(c["ids"][i:i + 1]) for i in range(len(c["ids"]))])
        assert np.abs(st - c["logits_steps"]).max() < 1e-5
        ids, _ = O.Model(s, 128).greedy(c["ids"], len(c["greedy"]))
        assert np.array_equal(ids, c["greedy"])


@pytest.mark.parametrize("file,tag", [("q8_0", "qwen35"), ("text-q8_0", "qwen35-text")])
def test_oracle_qwen35_q8_0_vs_transformers(file, tag):
    # Q8_0 weights (ssm_alpha/ssm_beta and the head too) against the float32
    # logits: the reference's own bound (test.infer.qwen35.pas:1081-1086)
    s = H.GgufSpec(os.path.join(GG, "qwen35", file + ".gguf"))
    for c in cases(tag):
        for f32 in (False, True):
            lg = O.Model(s, 128, f32=f32).forward(c["ids"], all_logits=True)
            assert np.abs(lg - c["logits"]).max() < 0.5
            assert cos(lg, c["logits"]) > 0.99


def test_oracle_recurrent_truncate():
    # a recurrent state holds the whole sequence: back to 0 only
    s = H.GgufSpec(os.path.join(GG, "qwen35", "bf16.gguf"))
    m = O.Model(s, 64)
    ids = np.arange(3, 12, dtype=np.int32)
    a = m.forward(ids)
    with pytest.raises(ValueError):
        m.truncate(4)
    m.truncate(len(ids))
    m.truncate(0)
    assert np.array_equal(m.forward(ids), a)


# ------------------------------------------------------------ closed forms
def test_gate_sigmoid_closed_form():
    a = np.array([1.5, -2.0, 3.0, 0.25, 7.0], np.float32)
    g = np.array([0.0, 2.0, -3.0, -150.0, 40.0], np.float32)
    want = a.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    want[3] = 0.0  # below -100: 0
    got = O.gate_sigmoid(a, g)
    assert np.allclose(got, want, rtol=2e-7, atol=0)


def delta_rule_f64(qkv, kh, vh, dk, dv, group, beta, decay, state):
    """S_t = g S + k (b (v - (g S) k))^T per value head, o = S_t q, in float64."""
    S = state.astype(np.float64).reshape(vh, dv, dk).copy()
    kd = kh * dk
    y = np.zeros((qkv.shape[0], vh * dv))
    for t in range(qkv.shape[0]):
        for h in range(vh):
            off = ((h // group) % kh) * dk
            q = qkv[t, off:off + dk].astype(np.float64)
            k = qkv[t, kd + off:kd + off + dk].astype(np.float64)
            v = qkv[t, 2 * kd + h * dv:2 * kd + (h + 1) * dv].astype(np.float64)
            Sd = S[h] * decay[t, h]
            S[h] = Sd + np.outer(beta[t, h] * (v - Sd @ k), k)
            y[t, h * dv:(h + 1) * dv] = S[h] @ q
    return y, S.reshape(state.shape)


@pytest.mark.parametrize("kh,vh,group", [(2, 2, 1), (2, 4, 2), (2, 4, 1), (1, 3, 3)])
def test_delta_rule_closed_form(kh, vh, group):
    rng = np.random.default_rng(kh * 10 + vh + group)
    dk, dv, rows = 16, 8, 6
    cd = 2 * kh * dk + vh * dv
    qkv = rng.standard_normal((rows, cd)).astype(np.float32) * 0.5
    beta = rng.uniform(0.1, 0.9, (rows, vh)).astype(np.float32)
    decay = rng.uniform(0.5, 1.0, (rows, vh)).astype(np.float32)
    state = rng.standard_normal((vh, dv, dk)).astype(np.float32) * 0.1
    y, st = O.delta_rule(qkv, kh, vh, dk, dv, group, beta, decay, state)
    yw, sw = delta_rule_f64(qkv, kh, vh, dk, dv, group, beta, decay, state)
    assert np.abs(y - yw).max() < 1e-5 * max(1.0, np.abs(yw).max())
    assert np.abs(st - sw).max() < 1e-5 * max(1.0, np.abs(sw).max())


def test_delta_rule_writes_the_value():
    # decay 1, beta 1, a unit key: the state then maps the key to the value
    # exactly, whatever it held (the delta rule's defining property); the
    # query equal to the key reads the value back
    rng = np.random.default_rng(7)
    dk, dv = 16, 8
    k = rng.standard_normal(dk)
    k = (k / np.linalg.norm(k)).astype(np.float32)
    v = rng.standard_normal(dv).astype(np.float32)
    qkv = np.concatenate([k, k, v])[None, :].astype(np.float32)
    state = rng.standard_normal((1, dv, dk)).astype(np.float32)
    y, _ = O.delta_rule(qkv, 1, 1, dk, dv, 1, np.ones((1, 1), np.float32),
                        np.ones((1, 1), np.float32), state)
    assert np.abs(y[0] - v).max() < 1e-5


def test_delta_prep_closed_form():
    rng = np.random.default_rng(3)
    kh, vh, dk, dv, kw, rows = 2, 4, 16, 8, 4, 5
    cd, vd = 2 * kh * dk + vh * dv, vh * dv
    qkv = rng.standard_normal((rows, cd)).astype(np.float32)
    beta = rng.standard_normal((rows, vh)).astype(np.float32) * 3
    beta[0, 0] = -200.0  # below -100: sigmoid 0
    decay = rng.standard_normal((rows, vh)).astype(np.float32) * 4
    decay[1, 1] = 30.0   # beyond 20: softplus(x) = x
    decay[2, 2] = -40.0  # exp(x) < 1e-6: log1p
    z = rng.standard_normal((rows, vd)).astype(np.float32)
    conv = rng.standard_normal((cd, kw - 1)).astype(np.float32)
    w = rng.standard_normal((cd, kw)).astype(np.float32) * 0.5
    dtb = rng.standard_normal(vh).astype(np.float32)
    nega = -np.exp(rng.standard_normal(vh)).astype(np.float32)
    q2, b2, d2, z2, c2 = O.delta_prep(qkv, beta, decay, z, conv, w, dtb, nega, kh, vh, dk, dv, kw)
    # the causal convolution over [the kept inputs | the new rows], silu
    full = np.concatenate([conv.T.astype(np.float64), qkv.astype(np.float64)])
    x = np.stack([(full[t:t + kw] * w.T.astype(np.float64)).sum(0) for t in range(rows)])
    x = x / (1 + np.exp(-x))
    assert np.array_equal(c2, qkv[-(kw - 1):].T)
    # q and k heads L2-normed, q times dk^-0.5
    for i in range(2 * kh):
        sl = slice(i * dk, (i + 1) * dk)
        xi = x[:, sl] / np.sqrt((x[:, sl] ** 2).sum(1, keepdims=True) + 1e-6)
        if i < kh:
            xi = xi / np.sqrt(dk)
        assert np.allclose(q2[:, sl], xi, rtol=1e-5, atol=1e-6)
    assert np.allclose(q2[:, 2 * kh * dk:], x[:, 2 * kh * dk:], rtol=1e-5, atol=1e-6)
    bw = 1 / (1 + np.exp(-beta.astype(np.float64)))
    bw[0, 0] = 0
    assert np.allclose(b2, bw, rtol=1e-6, atol=0)
    a = decay.astype(np.float64) + dtb
    sp = np.where(a > 20, a, np.log1p(np.exp(np.minimum(a, 20))))
    assert np.allclose(d2, np.exp(nega * sp), rtol=1e-5, atol=1e-30)
    zd = z.astype(np.float64)
    assert np.allclose(z2, zd / (1 + np.exp(-zd)), rtol=1e-6, atol=1e-7)
