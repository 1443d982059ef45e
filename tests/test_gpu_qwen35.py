"""Qwen3.5 on the device (deltanet.hip and the gated attention of model.cpp):
the qwen35 GGUF files of the reference's tests (tiny-qwen35 and its text
variant: Gated DeltaNet layers, 2 or 4 value heads over 2 key heads, the tiled
llama.cpp order, convolutions of 4 and 3, a quarter or half of each head
rotating, gated full attention) against the CPU oracle on the same mapped bytes
(logits within 1e-5 relative; greedy token-identical) and against the float32
logits transformers wrote (the reference's device bound, test.infer.cuda.pas
Qwen3.5 cases); the recurrent state carried across prompt chunks and decode
steps, and the contexts' rules for it (Reuse / Truncate back to 0 only)."""
import os

import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O

pytestmark = pytest.mark.gpu

GG = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gguf")
EXP = np.load(os.path.join(GG, "expected.npz"))

FILES = [("bf16", "qwen35"), ("q8_0", "qwen35"), ("text-bf16", "qwen35-text"),
         ("text-q8_0", "qwen35-text")]


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    yield c
    c.close()


def cases(tag):
    out, k = [], 0
    while f"{tag}/case{k}.ids" in EXP.files:
        out.append({f: EXP[f"{tag}/case{k}.{f}"] for f in ("ids", "logits", "logits_steps", "greedy")})
        k += 1
    return out


def spec(file):
    return H.GgufSpec(os.path.join(GG, "qwen35", file + ".gguf"))


def rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


@pytest.mark.parametrize("mode", [H.MODE_Q8, H.MODE_F32])
@pytest.mark.parametrize("file,tag", FILES)
def test_qwen35_device_matches_oracle(ctx, file, tag, mode):
    s = spec(file)
    for k, c in enumerate(cases(tag)):
        print(file, "mode", mode, "case", k, flush=True)
        dev = H.Model(ctx, s, mode=mode, max_tokens=96)
        cpu = O.Model(s, 96, f32=(mode == H.MODE_F32))
        a = dev.forward(c["ids"], all_logits=True)
        b = cpu.forward(c["ids"], all_logits=True)
        assert rel(a, b) < 1e-5, (k, rel(a, b))
        # greedy: the prompt, then 24 decode steps on the graph (one token
        # at a time through the recurrent state)
        dev.reset()
        got = dev.greedy(c["ids"], 24)
        ref, margins = O.Model(s, 96, f32=(mode == H.MODE_F32)).greedy(c["ids"], 24)
        print("  min margin", float(margins.min()), flush=True)
        assert np.array_equal(got, ref), (k, got, ref, margins)
        dev.close()
        cpu.close()


@pytest.mark.parametrize("file,tag", [("bf16", "qwen35"), ("text-bf16", "qwen35-text")])
def test_qwen35_device_vs_transformers(ctx, file, tag):
    # BF16 widened exactly, the F32 arithmetic: transformers' float32 logits
    # in one pass and one token at a time, and its greedy tokens
    s = spec(file)
    for c in cases(tag):
        dev = H.Model(ctx, s, mode=H.MODE_F32, max_tokens=96)
        lg = dev.forward(c["ids"], all_logits=True)
        assert rel(lg, c["logits"]) < 1e-5
        dev.reset()
        st = np.stack([dev.forward(c["ids"][i:i + 1]) for i in range(len(c["ids"]))])
        assert rel(st, c["logits_steps"]) < 1e-5
        dev.reset()
        assert np.array_equal(dev.greedy(c["ids"], len(c["greedy"])), c["greedy"])
        dev.close()


@pytest.mark.parametrize("rows", [1, 3, 7])
def test_qwen35_state_across_chunks(ctx, rows):
    # a prompt in chunks of `rows`: the convolution inputs and the state carry
    # from chunk to chunk, the logits are those of one pass
    s = spec("text-q8_0")
    c = cases("qwen35-text")[2]
    one = H.Model(ctx, s, max_tokens=64)
    want = one.forward(c["ids"], all_logits=True)
    dev = H.Model(ctx, s, max_tokens=64)
    dev.chunk(rows)
    got = dev.forward(c["ids"], all_logits=True)
    assert rel(got, want) < 1e-6
    one.close()
    dev.close()


def test_qwen35_contexts_reuse_and_truncate(ctx):
    # a recurrent state holds the whole sequence: Reuse keeps all the cached
    # tokens or none, Truncate goes back to 0 only; two contexts of one model
    # keep their own states
    s = spec("q8_0")
    c = cases("qwen35")[2]
    ids = c["ids"]
    m = H.Model(ctx, s, max_tokens=64)
    a, b = m.new_context(), m.new_context()
    la = a.forward(ids[:20])
    b.forward(ids[:9])
    assert rel(a.forward(ids[20:21]), m.new_context().forward(ids[:21])) < 1e-6
    # the whole cache is a prefix of the prompt: kept
    assert a.reuse(np.concatenate([ids[:21], [5, 6]])) == 21
    # a shorter common start: nothing kept, the state starts again
    assert b.reuse(np.concatenate([ids[:5], [7, 8]])) == 0
    assert b.length()[0] == 0
    with pytest.raises(H.HipError):
        a.truncate(10)
    a.truncate(0)
    assert rel(a.forward(ids[:20]), la) < 1e-6
    a.close()
    b.close()
    m.close()


def test_qwen35_native_decode(ctx):
    # NativeDecode over a Qwen3.5 context: a second request that extends the
    # first conversation keeps the whole cached sequence; the greedy tokens
    # equal the CPU decoder's
    s = spec("text-q8_0")
    m = H.Model(ctx, s, max_tokens=128)
    cache = H.PromptCache(m, 1)
    p1 = cases("qwen35-text")[1]["ids"]
    t1, reused, _ = H.native_generate(cache, p1, 12)
    assert reused == 0
    want, _ = O.Model(s, 128).greedy(p1, 12)
    assert np.array_equal(t1, want)
    p2 = np.concatenate([p1, t1, [3, 4, 5]]).astype(np.int32)
    t2, reused, _ = H.native_generate(cache, p2, 8)
    assert reused == len(p1) + len(t1) - 1
    want2, _ = O.Model(s, 128).greedy(p2, 8)
    assert np.array_equal(t2, want2)
    cache.close()
    m.close()


def test_qwen35_real_widths(ctx):
    # Qwen3.5-0.8B's widths (16 key and value heads of 128: a state column of
    # 128 per wave, attention heads of 256) over 8 layers and a small
    # vocabulary: the device's greedy tokens are the CPU decoder's
    from infer_hip import models
    s = models.Spec(models.tiny("qwen35-0.8b-q8_0", layers=8, vocab=4096), seed=3)
    prompt = np.random.default_rng(5).integers(0, 4096, 90).astype(np.int32)
    dev = H.Model(ctx, s, max_tokens=160)
    got = dev.greedy(prompt, 32)
    ref, margins = O.Model(s, 160, threads=16).greedy(prompt, 32)
    print("min margin", float(margins.min()), flush=True)
    assert np.array_equal(got, ref)
    dev.close()


def test_qwen35_restore_points(ctx):
    # CheckpointId = T (a turn start): one forward of three turns keeps the
    # states before the second and third T; a branched conversation (the
    # third turn edited) resumes from the restore point before it and gives
    # the logits of a fresh pass; Truncate goes back to a restore point only;
    # decoded tokens (parts a fresh pass would not make) add none
    s = spec("text-q8_0")
    T = 7
    a = np.array([T, 11, 12, 13, 14, 15, T, 21, 22, 23, 24, T, 31, 32, 33], np.int32)
    m = H.Model(ctx, s, max_tokens=96)
    c = m.new_context()
    c.set_checkpoints(T, 4)
    c.forward(a)
    assert c.checkpoints() == [6, 11]
    b = np.concatenate([a[:12], [41, 42, 43]]).astype(np.int32)
    assert c.reuse(b) == 11
    assert c.checkpoints() == [6, 11]
    got = c.forward(b[11:])
    fresh = m.new_context()
    want = fresh.forward(b)
    assert rel(got, want) < 1e-6
    assert rel(want, O.Model(s, 96).forward(b)) < 1e-5
    # another turn from the cached branch, then back to the first restore point
    c.forward(np.array([T, 51, 52], np.int32))
    assert c.checkpoints() == [6, 11, 15]
    with pytest.raises(H.HipError):
        c.truncate(9)
    c.truncate(6)
    assert c.checkpoints() == [6]
    assert rel(c.forward(a[6:]), fresh_logits(m, a)) < 1e-6
    # decoded tokens: a part of one token not starting at T, unaligned
    c.decode(int(np.argmax(c.forward(np.array([T, 61], np.int32)))), 3)
    n = c.length()[0]
    c.forward(np.array([T, 71], np.int32))
    assert n not in c.checkpoints()
    # at most max_count kept, the oldest dropped
    c.set_checkpoints(T, 4)
    c.truncate(0)
    c.forward(np.array([T, 1, T, 2, T, 3, T, 4, T, 5, T, 6], np.int32))
    assert c.checkpoints() == [4, 6, 8, 10]
    c.close()
    fresh.close()
    m.close()


def test_qwen35_checkpoint_token_in_decode(ctx):
    """The CheckpointId token fed by a decode (graph) step: its own part, so
    an aligned context keeps the state before it (TDecoderModel.ForwardRows,
    decoder.pas:3221-3240), and that restore point gives the logits of a
    fresh pass. Drawn later in a decode, after steps that fed other tokens
    (parts a fresh pass would not make, CheckPart :1083-1101), it adds none,
    and the state goes on as a fresh pass of the same ids."""
    s = spec("text-q8_0")
    m = H.Model(ctx, s, max_tokens=96)
    P = np.array([3, 11, 12, 13], np.int32)
    T = 7
    c = m.new_context()
    c.set_checkpoints(T, 4)
    c.forward(P)
    d = c.decode(T, 3)  # feeds T, d[0], d[1]
    assert c.checkpoints() == [len(P)]
    c.truncate(len(P))
    tail = np.array([T, 21, 22], np.int32)
    got = c.forward(tail)
    want = fresh_logits(m, np.concatenate([P, tail]))
    assert rel(got, want) < 1e-6
    assert rel(want, O.Model(s, 96).forward(np.concatenate([P, tail]))) < 1e-5
    c.close()
    # a token drawn mid-decode as the checkpoint id
    probe = m.new_context()
    x = int(np.argmax(probe.forward(P)))
    g = probe.decode(x, 8).tolist()
    probe.close()
    fed = [x] + g
    j = next((i for i in range(2, len(fed)) if fed[i] not in fed[:i] and fed[i] not in P), None)
    if j is None:
        pytest.skip(f"the greedy tokens {fed} hold no new id after two steps")
    T2 = fed[j]
    c2 = m.new_context()
    c2.set_checkpoints(T2, 4)
    c2.forward(P)
    out = c2.decode(x, j + 2)  # feeds fed[0..j+1]: T2 at step j
    assert out.tolist() == g[:j + 2]
    assert c2.checkpoints() == []
    more = np.array([T2, 5], np.int32)
    got = c2.forward(more)
    assert c2.checkpoints() == []
    want = fresh_logits(m, np.concatenate([P, fed[:j + 2], more]).astype(np.int32))
    assert rel(got, want) < 1e-6
    c2.close()
    m.close()


def fresh_logits(m, ids):
    f = m.new_context()
    out = f.forward(ids)
    f.close()
    return out
