"""The TDecoderDevice surface of the device decoder (decoder.pas:907-928,
model.qwen3.cuda.pas:229-247), through the C-ABI, against the CPU oracle:

- ForwardEmbeds: embedding rows in place of ids give the logits of those ids,
  and the last row's final norm equals the oracle's;
- Reuse / Truncate: a context that keeps a common prefix and computes the
  rest gives the logits and greedy tokens of a fresh pass;
- several contexts of one model (NewDeviceContext) interleaved, each with its
  own cache and decode graph, each token-identical to its own oracle run;
- the KV cache growing from nothing past several doublings (Prepare), also in
  the middle of a decode, token-identical to the oracle.
"""
import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O
from infer_hip import models

pytestmark = pytest.mark.gpu

FAMILIES = [
    ("qwen3-0.6b-q4_k_m", dict(layers=2, vocab=2048, hidden=512, heads=8, kv_heads=4,
                               head_dim=64, ffn=768)),
    ("qwen3-30b-a3b-q4_k_m", dict(layers=2, vocab=2048, hidden=512, heads=8, kv_heads=2,
                                  head_dim=128, experts=16, experts_used=4, expert_ffn=256)),
    ("gpt-oss-20b-mxfp4", dict(layers=2, vocab=2048, hidden=512, heads=8, kv_heads=2,
                               head_dim=64, experts=8, experts_used=2, expert_ffn=512,
                               window=16)),
]


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    yield c
    c.close()


def rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


@pytest.mark.parametrize("name,over", FAMILIES)
def test_forward_embeds_equals_ids(ctx, name, over):
    spec = models.Spec(models.tiny(name, **over), seed=71)
    d = spec.struct
    ids = np.random.default_rng(3).integers(0, spec.vocab, 9).astype(np.int32)
    # the embedding table is the Spec's first host tensor
    emb = O.dequant(spec.keep[0], d.embed.dtype, d.vocab, d.hidden)[ids]
    model = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=True, max_tokens=64)
    a = model.new_context()
    b = model.new_context()
    la = a.forward(ids)
    lb, nb = b.forward_embeds(emb, normed=True)
    # the same rows through the same kernels: the same bits
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    cpu = O.Model(spec, 64, kv_f16=True)
    lc, nc = cpu.forward_embeds(emb, d.hidden, normed=True)
    assert rel(lb, lc) < 1e-5 and rel(nb, nc) < 1e-5
    # one more row each (the one-row path), its norm too
    row = emb[:1] * 0.5
    lb1, nb1 = b.forward_embeds(row, normed=True)
    lc1, nc1 = cpu.forward_embeds(row, d.hidden, normed=True)
    assert rel(lb1, lc1) < 1e-5 and rel(nb1, nc1) < 1e-5
    # a position fed a row matches no id: Reuse keeps none of them
    assert b.reuse(np.concatenate([ids, [1, 2]])) == 0
    with pytest.raises(H.HipError):
        b.forward_embeds(row, head=1)  # one head only
    cpu.close()
    model.close()


@pytest.mark.parametrize("name,over", FAMILIES)
def test_reuse_and_truncate_match_a_fresh_pass(ctx, name, over):
    spec = models.Spec(models.tiny(name, **over), seed=73)
    rng = np.random.default_rng(5)
    first = rng.integers(0, spec.vocab, 40).astype(np.int32)
    second = np.concatenate([first[:25], rng.integers(0, spec.vocab, 15).astype(np.int32)])
    model = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=True, max_tokens=128)
    s = model.new_context()
    s.forward(first)
    kept = s.reuse(second)
    assert kept == 25 and s.length()[0] == 25
    got = s.forward(second[kept:])
    cpu = O.Model(spec, 128, kv_f16=True)
    ref = cpu.forward(second)
    assert rel(got, ref) < 1e-5
    # the whole prompt again: at most count - 1 tokens are kept
    assert s.reuse(second) == len(second) - 1
    got2 = s.forward(second[-1:])
    assert rel(got2, ref) < 1e-5
    # greedy continuation after a truncate equals the oracle's from that point
    s.truncate(30)
    cpu.truncate(30)
    g = s.greedy(second[30:], 16)
    r, _ = cpu.greedy(second[30:], 16)
    assert np.array_equal(g, r), (g, r)
    with pytest.raises(H.HipError):
        s.truncate(10_000)
    cpu.close()
    model.close()


@pytest.mark.parametrize("name,over", FAMILIES)
def test_contexts_interleaved(ctx, name, over):
    spec = models.Spec(models.tiny(name, **over), seed=79)
    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, spec.vocab, n).astype(np.int32) for n in (12, 30, 7)]
    model = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=True, max_tokens=64)
    cs = [model.new_context() for _ in prompts]
    refs = []
    for p in prompts:
        cpu = O.Model(spec, 128, kv_f16=True)
        r, _ = cpu.greedy(p, 24)
        refs.append(r)
        cpu.close()
    # each context's prompt, then its decode in turns of 4 steps
    outs = [[int(np.argmax(c.forward(p)))] for c, p in zip(cs, prompts)]
    for _ in range(6):
        for c, o in zip(cs, outs):
            o.extend(c.decode(o[-1], 4).tolist())
    for o, r in zip(outs, refs):
        assert np.array_equal(np.array(o[:24], np.int32), r), (o[:24], r)
    # the model's own context is unaffected by the others
    own = model.greedy(prompts[0], 8)
    assert np.array_equal(own, refs[0][:8])
    for c in cs:
        c.close()
    model.close()


@pytest.mark.parametrize("name,over", FAMILIES)
def test_cache_grows_from_empty(ctx, name, over):
    spec = models.Spec(models.tiny(name, **over), seed=83)
    prompt = np.random.default_rng(13).integers(0, spec.vocab, 150).astype(np.int32)
    model = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=True, max_tokens=16)
    s = model.new_context()
    assert s.length() == (0, 0)
    # 60 tokens: a cache of 75; the decode then grows it under the graph
    s.forward(prompt[:60])
    n, cap = s.length()
    assert n == 60 and 60 <= cap < 150
    nxt = int(np.argmax(s.forward(prompt[60:150])))
    ids = [nxt] + s.decode(nxt, 100).tolist()
    n2, cap2 = s.length()
    assert n2 == 250 and cap2 >= 250 and cap2 > cap
    cpu = O.Model(spec, 300, kv_f16=True)
    r, margins = cpu.greedy(prompt, 101)
    assert np.array_equal(np.array(ids, np.int32), r), (np.nonzero(np.array(ids) != r)[0][:4], margins)
    # the model's own context (16 tokens up front) grows too
    own = model.greedy(prompt[:40], 20)
    cpu2 = O.Model(spec, 300, kv_f16=True)
    r2, _ = cpu2.greedy(prompt[:40], 20)
    assert np.array_equal(own, r2)
    cpu.close()
    cpu2.close()
    s.close()
    model.close()
