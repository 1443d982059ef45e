"""TNativeLlmClient's device side (src/mormot.ai.llm.native.pas): NativeDecode
(:2135-2185) on a context and TNativePromptCache (:2192-2350), through the
C-ABI, against the CPU decoder (the oracle) drawing from its own logits.

- greedy and sampled requests give the oracle's tokens (a fresh sampler per
  request: the same seed, the same draws);
- a stop id ends the request at its first draw, and the context then holds
  the prompt and every drawn token but the last (that one is not fed);
- draws among the first draw_ids rows (a tokenizer with fewer ids);
- the context limit: a prompt beyond it is refused, max_new cut to fit;
- the prompt cache hands the context of a conversation back to its next turn
  (a hit, its tokens reused) with the tokens of a fresh context, frees the
  least recently used when full, and Clear / SetSlots free idle contexts."""
import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O
from infer_hip import models

pytestmark = pytest.mark.gpu

SPEC_KW = dict(layers=2, vocab=2048, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512)


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def spec():
    return models.Spec(models.tiny("qwen3-0.6b-q8_0", **SPEC_KW), seed=7)


def oracle_tokens(spec, prompt, max_new, kw=None, stop=(), ids=0):
    cpu = O.Model(spec, len(prompt) + max_new + 4)
    smp = O.Sampler(**kw) if kw else None
    lg = cpu.forward(prompt)
    out = []
    while True:
        row = lg[:ids] if ids else lg
        t = smp.next(row) if smp else O.argmax(row)
        out.append(t)
        if t in stop or len(out) == max_new:
            break
        lg = cpu.forward([t])
    cpu.close()
    return out


def test_native_decode_greedy_and_stop(ctx, spec):
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=128)
    prompt = np.random.default_rng(1).integers(0, spec.vocab, 12).astype(np.int32)
    ref = oracle_tokens(spec, prompt, 24)
    c = dev.new_context()
    got, reused, stopped = c.native_decode(prompt, 24)
    assert list(got) == ref and reused == 0 and not stopped
    assert c.length()[0] == len(prompt) + len(got) - 1
    # a stop id: the request ends at its first draw
    stop = ref[6]
    first = ref.index(stop)
    c2 = dev.new_context()
    got, _, stopped = c2.native_decode(prompt, 24, stop=(stop, -5))
    assert stopped and list(got) == ref[:first + 1]
    assert c2.length()[0] == len(prompt) + first
    c.close(); c2.close(); dev.close()


def test_native_decode_sampled_and_draw_ids(ctx, spec):
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=128)
    prompt = np.random.default_rng(2).integers(0, spec.vocab, 10).astype(np.int32)
    kw = dict(temperature=0.8, top_k=40, top_p=0.95, seed=99)
    ref = oracle_tokens(spec, prompt, 16, kw)
    for _ in range(2):  # a fresh sampler per request: the same draws
        c = dev.new_context()
        got, _, _ = c.native_decode(prompt, 16, kw)
        c.close()
        assert list(got) == ref
    # draws among the first 1000 rows only
    ref_ids = oracle_tokens(spec, prompt, 16, kw, ids=1000)
    c = dev.new_context()
    got, _, _ = c.native_decode(prompt, 16, kw, draw_ids=1000)
    assert list(got) == ref_ids and max(got) < 1000
    # greedy again after sampled requests
    got, _, _ = dev.new_context().native_decode(prompt, 8)
    assert list(got) == oracle_tokens(spec, prompt, 8)
    c.close(); dev.close()


def test_native_decode_two_threads_keep_their_settings(ctx, spec):
    """Two requests with different sampling settings on two contexts of one
    model, from two threads at once: each draws its own settings' tokens
    (the sampler is set up and used under one hold of the device lock)."""
    import threading
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=128)
    prompt = np.random.default_rng(5).integers(0, spec.vocab, 10).astype(np.int32)
    kws = [dict(temperature=0.8, top_k=40, top_p=0.95, seed=11),
           dict(temperature=1.3, top_k=8, min_p=0.01, seed=5), None]
    refs = [oracle_tokens(spec, prompt, 12, kw) for kw in kws]
    ctxs = [dev.new_context() for _ in kws]
    got = [[] for _ in kws]
    errors = []

    def run(i):
        try:
            for _ in range(4):
                toks, _, _ = ctxs[i].native_decode(prompt, 12, kws[i])
                got[i].append(list(toks))
        except Exception as e:  # reported by the main thread
            errors.append(e)

    th = [threading.Thread(target=run, args=(i,)) for i in range(len(kws))]
    for t in th:
        t.start()
    for t in th:
        t.join()
    for c in ctxs:
        c.close()
    dev.close()
    assert not errors, errors
    for i, ref in enumerate(refs):
        assert all(g == ref for g in got[i]), (i, got[i], ref)


def test_native_decode_limits(ctx, spec):
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=128)
    prompt = np.random.default_rng(3).integers(0, spec.vocab, 10).astype(np.int32)
    c = dev.new_context()
    with pytest.raises(H.HipError):
        c.native_decode(prompt, 4, max_context=9)  # the prompt exceeds the context
    with pytest.raises(H.HipError):
        c.native_decode(prompt[:0], 4)  # empty prompt
    with pytest.raises(H.HipError):
        c.native_decode(prompt, 0)  # no new token
    got, _, _ = c.native_decode(prompt, 50, max_context=13)  # cut to 13 - 10 + 1
    assert len(got) == 4 and list(got) == oracle_tokens(spec, prompt, 4)
    c.close(); dev.close()


def test_prompt_cache_conversation(ctx, spec):
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=128)
    rng = np.random.default_rng(4)
    p1 = rng.integers(0, spec.vocab, 14).astype(np.int32)
    cache = H.PromptCache(dev, slots=2)
    a, reused, _ = H.native_generate(cache, p1, 10)
    assert reused == 0 and list(a) == oracle_tokens(spec, p1, 10)
    # the next turn: the first turn, its answer, a new question
    p2 = np.concatenate([p1, a, rng.integers(0, spec.vocab, 5).astype(np.int32)])
    b, reused, _ = H.native_generate(cache, p2, 10)
    assert reused == len(p1) + len(a) - 1  # the last drawn token was never fed
    assert list(b) == oracle_tokens(spec, p2, 10)
    st = cache.stats()
    assert st["requests"] == 2 and st["hits"] == 1 and st["reused"] == reused and st["idle"] == 1
    # an unrelated prompt: a new context (one slot free), then the cache full
    p3 = rng.integers(0, spec.vocab, 9).astype(np.int32)
    c3, reused, _ = H.native_generate(cache, p3, 6)
    assert reused == 0 and list(c3) == oracle_tokens(spec, p3, 6)
    assert cache.stats()["idle"] == 2
    # full and nothing shared: the least recently used context is taken over
    p4 = rng.integers(0, spec.vocab, 11).astype(np.int32)
    d4, reused, _ = H.native_generate(cache, p4, 6)
    assert reused == 0 and list(d4) == oracle_tokens(spec, p4, 6)
    assert cache.stats()["idle"] == 2
    # the second conversation goes on from its cached context
    p5 = np.concatenate([p3, c3, p4[:3]])
    e5, reused, _ = H.native_generate(cache, p5, 5)
    assert reused == len(p3) + len(c3) - 1 and list(e5) == oracle_tokens(spec, p5, 5)
    cache.set_slots(1)
    assert cache.stats()["idle"] == 1
    cache.clear()
    assert cache.stats()["idle"] == 0
    # no slot: every context freed after its request
    cache.set_slots(0)
    H.native_generate(cache, p1, 3)
    assert cache.stats()["idle"] == 0
    cache.close(); dev.close()
