"""The AVX2 restatement of TInferCpuFastBackend (oracle/fast.c), the timed CPU
baseline, pinned (CPU only):

- K-quant Linear: the exact super-block sums and DotK's double arithmetic,
  so the bits of orc_linear (which is pinned by the golden linear/y) for
  every row count (pairs of rows and a last single one) and tile edge;
- every format against the reference's golden linear/y at its own tolerances
  (the float lanes of Q8DotF32x4x2 are tolerance-pinned in the reference too,
  test.infer.gguf.pas:450-451, :801);
- F32 weights against the double Linear within float-lane rounding;
- the fast attention against the double CausalRows brute force;
- a tiny decoder on the fast path gives the oracle's greedy tokens.
"""
import numpy as np
import pytest

import oracle_lib as O
from golden_io import GoldenSet, compare
from infer_hip import models

pytestmark = pytest.mark.skipif(not O.fast_available(), reason="no AVX2/FMA/F16C on this host")

import infer_hip as H  # noqa: E402


@pytest.mark.parametrize("dtype", [O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("rows", [1, 2, 3, 5])
def test_kquant_bits_of_the_oracle(dtype, rows):
    nin, out = 1024, 37  # a tile of 16, a second one and a partial third
    w = H.synth_normal(dtype, out, nin, 5 + rows, 0.05)
    x = np.random.default_rng(rows).standard_normal((rows, nin)).astype(np.float32)
    b = np.random.default_rng(9).standard_normal(out).astype(np.float32)
    a = O.fast_linear(x, w, dtype, out, b, threads=4)
    r = O.linear(x, w, dtype, out, b)
    assert np.array_equal(a.view(np.uint32), r.view(np.uint32))


LINEAR = [("q8", "linear/weight", "linear/y", O.Q8_0, 1e-5, 1e-5),
          ("q4", "linear/weight", "linear/y", O.Q4_0, 1e-5, 1e-5),
          ("q5", "linear/weight", "linear/y", O.Q5_0, 1e-5, 1e-5),
          ("q51", "linear/weight", "linear/y", O.Q5_1, 2e-3, 2e-4),
          ("mxfp4", "linear/weight", "linear/y", O.MXFP4, 1e-5, 1e-5),
          ("qk", "q4_K/weight", "q4_K/y", O.Q4_K, 1e-4, 1e-5),
          ("qk", "q6_K/weight", "q6_K/y", O.Q6_K, 1e-4, 1e-5)]


@pytest.mark.parametrize("name,wkey,ykey,dtype,atol,rtol", LINEAR)
def test_fast_linear_like_ggml(name, wkey, ykey, dtype, atol, rtol):
    g = GoldenSet(name)
    x, b, w, y = g["linear/x"], g["linear/bias"], g[wkey], g[ykey]
    mine = O.fast_linear(x, np.ascontiguousarray(w), dtype, b.size, b, threads=3)
    ok, err = compare(mine, y, atol, rtol)
    assert ok, err


@pytest.mark.parametrize("dtype", [O.F32, O.BF16])
def test_fast_float_weights(dtype):
    nin, out, rows = 512, 40, 3
    w = H.synth_normal(dtype, out, nin, 3, 0.05)
    x = np.random.default_rng(2).standard_normal((rows, nin)).astype(np.float32)
    a = O.fast_linear(x, w, dtype, out, threads=2)
    r = O.linear(x, w, dtype, out)
    assert np.abs(a - r).max() <= 1e-5 * np.abs(r).max()


def test_fast_attention_brute_force():
    rng = np.random.default_rng(4)
    heads, kvh, hd, past, rows = 4, 2, 32, 150, 5
    T = past + rows
    q = rng.standard_normal((rows, heads * hd)).astype(np.float32)
    keys = rng.standard_normal((T, kvh * hd)).astype(np.float32)
    values = rng.standard_normal((T, kvh * hd)).astype(np.float32)
    sinks = rng.standard_normal(heads).astype(np.float32)
    for window, sk in ((0, None), (64, sinks)):
        y = np.empty_like(q)
        O.lib().orc_fast_attention(q.ctypes.data, rows, heads, hd, keys.ctypes.data,
                                   values.ctypes.data, past, kvh, y.ctypes.data, window,
                                   None if sk is None else sk.ctypes.data, 3)
        r = O.causal_attention(q, heads, hd, keys, values, past, kvh, window, sk)
        assert np.abs(y - r).max() <= 1e-5 * np.abs(r).max()


@pytest.mark.parametrize("name,over", [
    ("qwen3-30b-a3b-q4_k_m", dict(layers=2, vocab=1024, hidden=512, heads=8, kv_heads=2,
                                  head_dim=64, experts=8, experts_used=2, expert_ffn=256)),
    ("qwen3-0.6b-q8_0", dict(layers=2, vocab=1024, hidden=256, heads=4, kv_heads=2,
                             head_dim=64, ffn=512)),
])
def test_fast_decoder_tokens(name, over):
    spec = models.Spec(models.tiny(name, **over), seed=17)
    prompt = np.random.default_rng(3).integers(0, spec.vocab, 20).astype(np.int32)
    a = O.Model(spec, 64, kv_f16=True, threads=4, fast=True)
    b = O.Model(spec, 64, kv_f16=True, threads=4)
    ga, _ = a.greedy(prompt, 16)
    gb, mb = b.greedy(prompt, 16)
    assert np.array_equal(ga, gb), (ga, gb, mb)
    a.close()
    b.close()
