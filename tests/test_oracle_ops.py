"""Pins of the oracle's non-Linear operations (CPU only), each against what the
mathematics or the published definition fixes, in a form a plausible
mistake (a dropped term, a wrong rounding point, a wrong tie or window rule,
a swapped half) fails:

- orc_rmsnorm: x / sqrt(mean(x^2) + eps) in double, the normed value rounded
  to single BEFORE the single multiply by w (backend.cpu.pas:1769-1795);
- orc_swiglu: silu(g) * u, and gpt-oss' clamped form (g clamped from above,
  u to [-limit, limit], (u + 1) * g * sigmoid(alpha * g)), each step in
  single (backend.cpu.pas:1797-1834; the published gpt-oss activation);
- orc_rope: rotate_half with angles in double, pairs (i, i + half)
  (backend.cpu.pas:1862-1888); partial rotation;
- orc_causal_attention: brute force softmax(q k^T / sqrt(d)) v in float64
  over T <= 8 keys, grouped heads, a window of the last `window` keys, and
  sinks as an extra softmax logit with no value (backend.cpu.pas:1305-1354);
- orc_route: softmax top-k, the LOWER id on an exact tie, the weights in
  pick order, each rounded to single, renormalised by their double sum
  (decoder.pas:2901-2949);
- orc_argmax: the first maximum, NaN skipped, -0 equal to +0, all-NaN gives 0
  (sampler.pas:123-160), against numpy's nanargmax;
- orc_rotary: cos/sin of pos * theta^(-2i/d) (decoder.pas:1735-1741,
  2539-2561) against float64 closed forms.

The composition of these into a decoder (orc_model_*) is pinned against an
independent float64 numpy decoder (np_model.py) in the F32 arithmetic, for
tiny models of every family.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from infer_hip import models

f32 = np.float32


def test_rmsnorm_rounds_normed_value_before_weight():
    rng = np.random.default_rng(1)
    for cols, scale, eps in ((1024, 1.0, 1e-6), (128, 1e-3, 1e-5), (2880, 30.0, 1e-5)):
        x = (rng.standard_normal((16, cols)) * scale).astype(f32)
        w = (rng.standard_normal(cols) * 0.5 + 1).astype(f32)
        y = O.rmsnorm(x, w, eps)
        x64 = x.astype(np.float64)
        inv = 1.0 / np.sqrt((x64 * x64).sum(axis=1, keepdims=True) / cols + eps)
        expect = (w * (x64 * inv).astype(f32)).astype(f32)
        assert np.array_equal(y.view(np.uint32), expect.view(np.uint32))
        # the other rounding order (w applied in double) differs: the pin bites
        other = (w.astype(np.float64) * x64 * inv).astype(f32)
        assert not np.array_equal(y, other)
    # eps inside the root: tiny inputs are damped, not blown up
    x = np.full((1, 64), 1e-4, f32)
    y = O.rmsnorm(x, np.ones(64, f32), 1e-6)
    assert abs(float(y[0, 0]) - 1e-4 / np.sqrt(1e-8 + 1e-6)) < 1e-6


def test_swiglu_plain_and_clamped():
    rng = np.random.default_rng(2)
    g = (rng.standard_normal(4096) * 4).astype(f32)
    u = (rng.standard_normal(4096) * 4).astype(f32)
    y = O.swiglu(g, u)
    g64 = g.astype(np.float64)
    expect = ((g64 / (1 + np.exp(-g64))).astype(f32) * u).astype(f32)
    assert np.array_equal(y.view(np.uint32), expect.view(np.uint32))
    alpha, limit = f32(1.702), f32(7.0)
    g = (rng.standard_normal(4096) * 8).astype(f32)
    u = (rng.standard_normal(4096) * 8).astype(f32)
    y = O.swiglu(g, u, float(alpha), float(limit))
    gc = np.minimum(g, limit)
    uc = np.clip(u, -limit, limit)
    b = (gc * alpha).astype(f32)
    s = (1 / (1 + np.exp(-b.astype(np.float64)))).astype(f32)
    expect = ((uc + f32(1)) * (gc * s).astype(f32)).astype(f32)
    assert np.array_equal(y.view(np.uint32), expect.view(np.uint32))
    # the gate is clamped from above only: a very negative gate stays (its silu ~ 0)
    y = O.swiglu(np.array([-50.0, 50.0], f32), np.array([100.0, -100.0], f32), 1.702, 7.0)
    assert y[0] == pytest.approx(8.0 * -50.0 / (1 + np.exp(1.702 * 50.0)), rel=1e-5)
    assert y[1] == pytest.approx(-6.0 * 7.0 / (1 + np.exp(-1.702 * 7.0)), rel=1e-6)


@pytest.mark.parametrize("rot", [0, 32])
def test_rope_rotate_half(rot):
    rng = np.random.default_rng(3)
    rows, heads, hd = 5, 3, 64
    half = (rot or hd) // 2
    x = rng.standard_normal((rows, heads * hd)).astype(f32)
    ang = rng.uniform(0, 50, (rows, half))
    cs, sn = np.cos(ang).astype(f32), np.sin(ang).astype(f32)
    y = O.rope(x, heads, hd, cs, sn, rot)
    t = x.reshape(rows, heads, hd).astype(np.float64)
    a, b = t[..., :half].copy(), t[..., half:2 * half].copy()
    c, s = cs[:, None, :].astype(np.float64), sn[:, None, :].astype(np.float64)
    e = t.copy()
    e[..., :half] = a * c - b * s
    e[..., half:2 * half] = b * c + a * s
    assert np.array_equal(y.reshape(rows, heads, hd), e.astype(f32))
    if rot:
        # the dimensions past the rotated ones are untouched
        assert np.array_equal(y.reshape(rows, heads, hd)[..., rot:], x.reshape(rows, heads, hd)[..., rot:])


def brute_attention(q, keys, values, heads, kvh, hd, past, window, sinks):
    rows = q.shape[0]
    y = np.zeros((rows, heads * hd))
    for r in range(rows):
        total = past + r + 1
        first = total - window if window > 0 and total > window else 0
        for h in range(heads):
            g = h // (heads // kvh)
            qv = q[r, h * hd:(h + 1) * hd].astype(np.float64)
            K = keys[first:total, g * hd:(g + 1) * hd].astype(np.float64)
            V = values[first:total, g * hd:(g + 1) * hd].astype(np.float64)
            s = K @ qv / np.sqrt(hd)
            logits = np.concatenate([s, [sinks[h]]]) if sinks is not None else s
            p = np.exp(logits - logits.max())
            p = p / p.sum()
            y[r, h * hd:(h + 1) * hd] = p[:len(s)] @ V
    return y


@pytest.mark.parametrize("past,rows,window,sinks", [(0, 8, 0, False), (3, 5, 0, False),
                                                     (2, 6, 3, False), (0, 8, 4, True),
                                                     (5, 3, 0, True), (0, 1, 0, False)])
def test_causal_attention_brute_force(past, rows, window, sinks):
    rng = np.random.default_rng(4 + past + rows)
    heads, kvh, hd = 4, 2, 16
    T = past + rows
    q = rng.standard_normal((rows, heads * hd)).astype(f32)
    keys = rng.standard_normal((T, kvh * hd)).astype(f32)
    values = rng.standard_normal((T, kvh * hd)).astype(f32)
    sk = rng.standard_normal(heads).astype(f32) if sinks else None
    y = O.causal_attention(q, heads, hd, keys, values, past, kvh, window, sk)
    e = brute_attention(q, keys, values, heads, kvh, hd, past, window, sk)
    assert np.abs(y - e).max() <= 1e-6 * max(1.0, np.abs(e).max())


def route_closed_form(lg, k, norm):
    order = sorted(range(len(lg)), key=lambda i: (-float(lg[i]), i))  # lower id on a tie
    top = order[:k]
    l64 = lg.astype(np.float64)
    p = np.exp(l64 - l64.max())
    p = p / p.sum()
    w = p[top].astype(f32)
    if norm:
        w = (w.astype(np.float64) / w.astype(np.float64).sum()).astype(f32)
    return np.array(top, np.int32), w


def test_route_ties_pick_order_and_renorm():
    rng = np.random.default_rng(5)
    for E, k in ((128, 8), (32, 4), (8, 8)):
        for norm in (True, False):
            lg = rng.standard_normal(E).astype(f32)
            lg[3] = lg[E - 1] = lg[E // 2] = lg.max() + 0.5  # a three-way tie at the top
            ids, w = O.route(lg, k, norm)
            eids, ew = route_closed_form(lg, k, norm)
            assert ids.tolist() == eids.tolist()
            assert ids[0] == 3 and ids[1] == E // 2 and ids[2] == E - 1
            assert np.allclose(w, ew, rtol=2e-7, atol=0)
            if norm:
                assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6
    # all equal: the k lowest ids, equal weights
    ids, w = O.route(np.zeros(16, f32), 4, True)
    assert ids.tolist() == [0, 1, 2, 3] and np.all(w == f32(0.25))


def test_route_nan_logits():
    # a NaN never compares greater: elsewhere than at id 0 it is never picked
    # while a number is left; the softmax sum turns NaN and so every weight
    lg = np.array([0.5, np.nan, 2.0, 1.0, -1.0], f32)
    ids, w = O.route(lg, 2, True)
    assert ids.tolist() == [2, 3] and np.all(np.isnan(w))
    # at id 0 it is the first candidate of each pick and nothing beats it
    lg = np.array([np.nan, 1.0, 3.0], f32)
    ids, w = O.route(lg, 2, False)
    assert ids.tolist() == [0, 2]


def test_argmax_rules():
    rng = np.random.default_rng(6)
    for _ in range(20):
        v = rng.standard_normal(1000).astype(f32)
        v[rng.integers(0, 1000, 30)] = np.nan
        v[rng.integers(0, 1000, 3)] = v[~np.isnan(v)].max()  # ties: the first wins
        assert O.argmax(v) == int(np.nanargmax(v))
    assert O.argmax(np.full(7, np.nan, f32)) == 0
    assert O.argmax(np.array([-0.0, 0.0, -0.0], f32)) == 0
    assert O.argmax(np.array([-1.0, -0.0, 0.0], f32)) == 1
    assert O.argmax(np.array([np.nan, -np.inf, -np.inf], f32)) == 1
    assert O.argmax(np.array([1.0, np.inf, np.nan, np.inf], f32)) == 1
    assert O.argmax(np.array([-3.0, -2.0, -2.5], f32)) == 1


def test_rotary_closed_form():
    cfg = models.tiny("qwen3-0.6b-q8_0", layers=1, vocab=64, hidden=64, heads=2, kv_heads=1,
                      head_dim=128, ffn=64)
    spec = models.Spec(cfg)
    d = spec.struct
    first, rows, hd = 1000, 4, 128
    cs = np.empty(rows * hd, f32)
    O.lib().orc_rotary(C.addressof(d), first, rows, cs.ctypes.data)
    half = hd // 2
    pos = np.arange(first, first + rows)[:, None].astype(np.float64)
    ang = pos * d.rope_theta ** (-2.0 * np.arange(half) / hd)
    assert np.allclose(cs[:rows * half].reshape(rows, half), np.cos(ang), atol=2e-4)
    assert np.allclose(cs[rows * half:].reshape(rows, half), np.sin(ang), atol=2e-4)


NP_MODELS = [
    ("qwen3-0.6b-q8_0", dict(layers=2, vocab=256, hidden=128, heads=4, kv_heads=2, head_dim=32,
                             ffn=256)),
    ("qwen3-0.6b-q4_k_m", dict(layers=2, vocab=256, hidden=256, heads=4, kv_heads=2,
                               head_dim=64, ffn=512)),
    ("qwen3-30b-a3b-q4_k_m", dict(layers=2, vocab=256, hidden=256, heads=4, kv_heads=2,
                                  head_dim=64, experts=8, experts_used=3, expert_ffn=256)),
    ("gpt-oss-20b-mxfp4", dict(layers=2, vocab=256, hidden=128, heads=4, kv_heads=2,
                               head_dim=32, experts=4, experts_used=2, expert_ffn=128,
                               window=4)),
]


@pytest.mark.parametrize("name,over", NP_MODELS)
def test_oracle_decoder_vs_numpy_float64(name, over):
    """orc_model_* (F32 arithmetic: dequantized weights, double sums) against
    np_model.NumpyModel, written from the architectures' formulas in float64."""
    import np_model

    spec = models.Spec(models.tiny(name, **over), seed=11, sigma=0.05)
    prompt = np.random.default_rng(7).integers(0, spec.vocab, 9).astype(np.int32)
    cpu = O.Model(spec, 32, f32=True)
    ref = np_model.NumpyModel(spec)
    a = cpu.forward(prompt)
    b = ref.forward(prompt)[-1]
    assert np.abs(a - b).max() <= 1e-5 * np.abs(b).max(), np.abs(a - b).max() / np.abs(b).max()
    # then two single-row steps (the cache, the window sliding past the prompt)
    for t in (3, 200):
        a = cpu.forward([t])
        b = ref.forward([t])[-1]
        assert np.abs(a - b).max() <= 1e-5 * np.abs(b).max()
    cpu.close()
