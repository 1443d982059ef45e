"""TInferSampler on the device (ihip_enqueue_sample, ihip_model_sampling)
against the CPU oracle of the same sampler: the same seed draws the same
tokens, draw for draw, for every warper and their combinations, at the
reference's small cases and at a real vocabulary; inside a replayed graph the
stream advances on the device; a sampled decode of a model draws the tokens
the CPU decoder draws from its own logits."""
import ctypes as C

import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O
from infer_hip import models

pytestmark = pytest.mark.gpu

NAN, NINF = np.uint32(0x7FC00000).view(np.float32), np.uint32(0xFF800000).view(np.float32)


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    yield c
    c.close()


def device_draws(ctx, logits, n, **kw):
    logits = np.ascontiguousarray(logits, np.float32)
    dl, do = ctx.array(logits), ctx.alloc(4)
    s = H.Sampler(ctx, logits.size, **kw)
    out = []
    for _ in range(n):
        s.enqueue(dl.ptr, logits.size, do.ptr)
        out.append(int(do.download(np.int32, 1)[0]))
    s.close()
    return out


def oracle_draws(logits, n, **kw):
    s = O.Sampler(**kw)
    out = [s.next(logits) for _ in range(n)]
    s.close()
    return out


def real_vocab(n=151936, seed=12345, spread=12.0):
    t, v = seed, np.empty(n, np.float32)
    for i in range(n):
        t = (t * 1103515245 + 12345) & 0x7FFFFFFF
        v[i] = (t / 0x7FFFFFFF) * spread - spread / 2
    return v


def peaked(n=151936, seed=3):
    # a language-model-like row: a few strong candidates over a long tail
    rng = np.random.default_rng(seed)
    v = rng.standard_normal(n).astype(np.float32) * 2
    v[rng.integers(0, n, 20)] += rng.uniform(6, 12, 20).astype(np.float32)
    return v


L3 = np.float32([0, np.log(2), np.log(4)])


def test_seed_42_on_the_device(ctx):
    assert device_draws(ctx, L3, 12, seed=42) == [2, 1, 1, 1, 0, 2, 1, 2, 1, 2, 1, 2]


SMALL = [
    (L3, dict(seed=1)), (L3, dict(temperature=0.5, seed=2)), (L3, dict(top_k=2, seed=3)),
    (L3, dict(top_p=0.5, seed=4)), (L3, dict(top_p=0.6, seed=5)), (L3, dict(min_p=0.4, seed=6)),
    (L3, dict(top_k=2, top_p=0.6, seed=7)),
    (np.zeros(3, np.float32), dict(top_k=2, seed=11)),
    (np.float32([0, 1e-20, -50]), dict(top_k=1, seed=15)),
    (np.float32([1, 1, NINF, NAN]), dict(seed=16)),
    (np.float32([NAN, 1, NINF, 1]), dict(seed=9)),
    (np.log(np.float32([0.5, 0.3, 0.2])).astype(np.float32), dict(top_p=0.6, min_p=0.5, seed=12)),
    (np.log(np.float32([0.5, 0.3, 0.2])).astype(np.float32), dict(temperature=1e-310, seed=14)),
]


@pytest.mark.parametrize("case", range(len(SMALL)))
def test_small_cases_draw_for_draw(ctx, case):
    logits, kw = SMALL[case]
    assert device_draws(ctx, logits, 300, **kw) == oracle_draws(logits, 300, **kw)


def test_whole_mass_and_beyond_the_finite_tokens(ctx):
    big = np.full(1002, np.log(1e-4), np.float32)
    big[0], big[1] = 0, np.log(0.5)
    assert device_draws(ctx, big, 300, top_p=0.65, seed=10) == oracle_draws(big, 300, top_p=0.65,
                                                                           seed=10)
    v = np.full(100, NINF, np.float32)
    v[0], v[7], v[50] = 0, np.log(2), np.log(4)
    assert device_draws(ctx, v, 300, top_k=50, seed=13) == oracle_draws(v, 300, top_k=50, seed=13)


BIG = [dict(temperature=0.7, top_p=0.9, seed=77), dict(top_k=50, seed=5),
       dict(temperature=0.8, min_p=0.05, seed=6), dict(top_k=40, top_p=0.95, min_p=0.02, seed=7),
       dict(temperature=1.0, seed=8), dict(temperature=0.6, top_k=20, top_p=0.8, seed=9),
       dict(temperature=1.3, top_p=0.5, seed=10), dict(top_k=1, seed=11)]


@pytest.mark.parametrize("kw", BIG)
@pytest.mark.parametrize("row", ["uniform", "peaked"])
def test_real_vocabulary_draw_for_draw(ctx, kw, row):
    v = real_vocab() if row == "uniform" else peaked()
    print(row, kw, flush=True)
    assert device_draws(ctx, v, 60, **kw) == oracle_draws(v, 60, **kw)


def test_draws_in_a_replayed_graph(ctx):
    # the stream lives on the device: each replay draws the next value
    v = peaked(seed=4)
    dl, do = ctx.array(v), ctx.alloc(4)
    s = H.Sampler(ctx, v.size, temperature=0.9, top_p=0.95, seed=21)
    H.check(H.lib().ihip_capture_begin(ctx.h), "capture")
    s.enqueue(dl.ptr, v.size, do.ptr)
    H.check(H.lib().ihip_capture_end(ctx.h, 3), "capture")
    got = []
    for _ in range(40):
        H.check(H.lib().ihip_graph_launch(ctx.h, 3), "launch")
        got.append(int(do.download(np.int32, 1)[0]))
    s.close()
    assert got == oracle_draws(v, 40, temperature=0.9, top_p=0.95, seed=21)


def test_refused_settings(ctx):
    for kw in (dict(top_p=0), dict(top_p=1.5), dict(min_p=1), dict(top_k=-1),
               dict(temperature=float("nan"))):
        with pytest.raises(H.HipError):
            H.Sampler(ctx, 16, **kw)


@pytest.mark.parametrize("name,over", [
    ("qwen3-0.6b-q8_0", dict(layers=2, vocab=2048, hidden=256, heads=4, kv_heads=2, head_dim=64,
                             ffn=512)),
    ("gpt-oss-20b-mxfp4", dict(layers=2, vocab=2048, hidden=512, heads=8, kv_heads=2,
                               head_dim=64, experts=8, experts_used=2, expert_ffn=512,
                               window=8))])
def test_model_sampled_decode(ctx, name, over):
    # the device decodes with its draws inside the graph; the CPU decoder draws
    # with the oracle sampler from its own logits: the same tokens
    spec = models.Spec(models.tiny(name, **over), seed=5)
    prompt = np.random.default_rng(6).integers(0, spec.vocab, 10).astype(np.int32)
    kw = dict(temperature=0.9, top_k=40, top_p=0.95, seed=123)
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=64)
    dev.sampling(**kw)
    got = dev.greedy(prompt, 20)
    cpu = O.Model(spec, 64)
    smp = O.Sampler(**kw)
    ref = []
    lg = cpu.forward(prompt)
    for _ in range(20):
        ref.append(smp.next(lg))
        lg = cpu.forward([ref[-1]])
    assert list(got) == ref
    # back to the argmax: the greedy tokens again
    dev.sampling()
    dev.reset()
    g1 = dev.greedy(prompt, 8)
    cpu2 = O.Model(spec, 64)
    g2, _ = cpu2.greedy(prompt, 8)
    assert np.array_equal(g1, g2)
    dev.close()
