"""The device decoder over llama.cpp GGUF files (the model files of the
reference's tests, tests/golden/gguf/): every file of qwen3, qwen3moe,
qwen2 (Qwen2.5: q/k/v biases, no head norm; the reference's device test is
tests/test.infer.cuda.pas:2240-2330) and gpt-oss against the CPU oracle on the same mapped bytes (tier 2: logits within
1e-5 relative; tier 3: greedy token-identical), and against the float32 logits
transformers wrote for the same weights, as the reference's device tests do
(tests/test.infer.cuda.pas:1560-1640, :1950-2010)."""
import os

import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O

pytestmark = pytest.mark.gpu

GG = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gguf")
EXP = np.load(os.path.join(GG, "expected.npz"))


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    yield c
    c.close()


def expected(tag):
    n = sum(1 for k in EXP.files if k.startswith(tag + "/") and k.endswith(".ids"))
    return [{f: EXP[f"{tag}/case{k}.{f}"] for f in ("ids", "logits", "greedy")
             if f"{tag}/case{k}.{f}" in EXP.files} for k in range(n)]


def rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


def cos(a, b):
    a, b = a.ravel().astype(np.float64), b.ravel().astype(np.float64)
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


FILES = [("qwen3/q8_0.gguf", "qwen3"), ("qwen3/q4_0.gguf", "qwen3"),
         ("qwen3/untied-f16.gguf", "qwen3-untied"), ("qwen3moe/q8_0.gguf", "qwen3moe"),
         ("qwen3moe/q4_0.gguf", "qwen3moe"), ("gpt-oss/bf16.gguf", "gpt-oss"),
         ("gpt-oss/q8_0.gguf", "gpt-oss"), ("qwen2/q8_0.gguf", "qwen2")]


@pytest.mark.parametrize("kv_f16", [False, True])
@pytest.mark.parametrize("file,tag", FILES)
def test_gguf_device_matches_oracle(ctx, file, tag, kv_f16):
    s = H.GgufSpec(os.path.join(GG, file))
    print(file, "kv_f16", kv_f16, flush=True)
    for k, c in enumerate(expected(tag)):
        dev = H.Model(ctx, s, mode=H.MODE_Q8, kv_f16=kv_f16, max_tokens=96)
        cpu = O.Model(s, 96, kv_f16=kv_f16)
        a = dev.forward(c["ids"], all_logits=True)
        b = cpu.forward(c["ids"], all_logits=True)
        assert rel(a, b) < 1e-5, (k, rel(a, b))
        dev.close()
        cpu.close()
        # greedy continuation: the prompt, then 24 decode steps on the graph
        dev = H.Model(ctx, s, mode=H.MODE_Q8, kv_f16=kv_f16, max_tokens=96)
        got = dev.greedy(c["ids"], 24)
        ref, margins = O.Model(s, 96, kv_f16=kv_f16).greedy(c["ids"], 24)
        print(" case", k, "min margin", float(margins.min()), flush=True)
        assert np.array_equal(got, ref), (k, got, ref, margins)
        dev.close()


@pytest.mark.parametrize("file,tag", [("qwen3/q8_0.gguf", "qwen3"),
                                      ("qwen3moe/q8_0.gguf", "qwen3moe"),
                                      ("qwen2/q8_0.gguf", "qwen2")])
def test_gguf_device_q8_0_vs_transformers(ctx, file, tag):
    # the Q8_0 file against the float32 logits of the BF16 checkpoint: within
    # the Q8_0 error, as the reference's device test bounds it (cosine 0.999)
    s = H.GgufSpec(os.path.join(GG, file))
    for c in expected(tag):
        dev = H.Model(ctx, s, mode=H.MODE_Q8, max_tokens=64)
        lg = dev.forward(c["ids"], all_logits=True)
        assert cos(lg, c["logits"]) > 0.999
        dev.close()


def test_gguf_device_gptoss_vs_transformers(ctx):
    # bf16.gguf with the checkpoint's SwiGLU limit (0.8): the F32 arithmetic on
    # the device gives transformers' logits within 1e-5 of the largest (the
    # reference's device bound is 1e-4, test.infer.cuda.pas:1541) and its
    # greedy tokens. Expert 1 of layer 0 holds a -0 block with the E8M0
    # exponent 255 (2^127): its zero values must stay exact zeros.
    s = H.GgufSpec(os.path.join(GG, "gpt-oss", "bf16.gguf"))
    s.struct.swiglu_limit = 0.8
    for c in expected("gpt-oss"):
        dev = H.Model(ctx, s, mode=H.MODE_F32, max_tokens=80)
        lg = dev.forward(c["ids"], all_logits=True)
        print("gpt-oss F32 vs transformers: relative", rel(lg, c["logits"]), flush=True)
        assert rel(lg, c["logits"]) < 1e-5
        dev.close()
        dev = H.Model(ctx, s, mode=H.MODE_F32, max_tokens=80)
        assert np.array_equal(dev.greedy(c["ids"], len(c["greedy"])), c["greedy"])
        dev.close()
