"""Tier 3: greedy decode on the device is token-identical to the CPU decoder
(the oracle restating TDecoderModel over TInferCpuBackend), for tiny models
of every family and for the BASELINE shapes. The device runs the Q8 (CPU)
arithmetic; each step's top-1/top-2 logit margin is recorded so a near tie
is reported, not hidden."""
import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O
from infer_hip import models

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    yield c
    c.close()


TINY = [
    ("qwen3-0.6b-q8_0", dict(layers=2, vocab=2048, hidden=256, heads=4, kv_heads=2, head_dim=64,
                             ffn=512)),
    ("qwen3-0.6b-q4_k_m", dict(layers=3, vocab=2048, hidden=512, heads=8, kv_heads=4,
                               head_dim=64, ffn=768)),
    ("qwen3-30b-a3b-q4_k_m", dict(layers=2, vocab=2048, hidden=512, heads=8, kv_heads=2,
                                  head_dim=128, experts=16, experts_used=4, expert_ffn=256)),
    ("gpt-oss-20b-mxfp4", dict(layers=4, vocab=2048, hidden=512, heads=8, kv_heads=2,
                               head_dim=64, experts=8, experts_used=2, expert_ffn=512,
                               window=8)),
    # SmolLM3-like: no head norms, every second layer without rotary
    # positions (NoPE), heads of 128 and of 64
    ("qwen3-0.6b-q8_0", dict(layers=4, vocab=2048, hidden=512, heads=4, kv_heads=2, head_dim=128,
                             ffn=768, qk_norm=False, no_rope_interval=2)),
    ("qwen3-0.6b-q4_k_m", dict(layers=4, vocab=2048, hidden=512, heads=8, kv_heads=4, head_dim=64,
                               ffn=768, qk_norm=False, no_rope_interval=2)),
]


@pytest.mark.parametrize("name,over", TINY)
def test_tiny_forward_logits_match_cpu(ctx, name, over):
    spec = models.Spec(models.tiny(name, **over), seed=21)
    prompt = np.random.default_rng(4).integers(0, spec.vocab, 12).astype(np.int32)
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=64)
    cpu = O.Model(spec, 64)
    a = dev.forward(prompt, all_logits=True)
    b = cpu.forward(prompt, all_logits=True)
    rel = np.abs(a - b).max() / np.abs(b).max()
    assert rel < 1e-5, rel
    # one decode row after the prompt
    a = dev.forward([5])
    b = cpu.forward([5])
    assert np.abs(a - b).max() / np.abs(b).max() < 1e-5
    dev.close()
    cpu.close()


@pytest.mark.parametrize("name,over", TINY)
@pytest.mark.parametrize("kv_f16", [False, True])
def test_tiny_greedy_token_identical(ctx, name, over, kv_f16):
    spec = models.Spec(models.tiny(name, **over), seed=33)
    prompt = np.random.default_rng(8).integers(0, spec.vocab, 16).astype(np.int32)
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=kv_f16, max_tokens=128)
    cpu = O.Model(spec, 128, kv_f16=kv_f16)
    got = dev.greedy(prompt, 48)
    ref, margins = cpu.greedy(prompt, 48)
    print(name, "kv_f16", kv_f16, "min margin", float(margins.min()), flush=True)
    assert np.array_equal(got, ref), (got, ref, margins)
    dev.close()
    cpu.close()


@pytest.mark.parametrize("name,prompt_len", [("qwen3-0.6b-q8_0", 32), ("qwen3-0.6b-q4_k_m", 32)])
def test_baseline_shape_greedy_64(ctx, name, prompt_len):
    # the full Qwen3-0.6B shape, 64 greedy tokens
    spec = models.Spec(models.CONFIGS[name], seed=1)
    prompt = np.random.default_rng(2024).integers(0, spec.vocab, prompt_len).astype(np.int32)
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=prompt_len + 80)
    got = dev.greedy(prompt, 64)
    cpu = O.Model(spec, prompt_len + 80, threads=16)
    ref, margins = cpu.greedy(prompt, 64)
    print(name, "min margin", float(margins.min()), "tokens", got[:8], flush=True)
    assert np.array_equal(got, ref), (np.nonzero(got != ref)[0][:5], margins)
    dev.close()
    cpu.close()


def test_nope_prompt_on_the_matrix_cores(ctx):
    # NoPE layers through a 96-row prefill (the GEMM and the prompt attention
    # on the f64 matrix cores) and the graph-replayed decode
    spec = models.Spec(models.tiny("qwen3-0.6b-q8_0", layers=4, vocab=2048, hidden=512, heads=4,
                                   kv_heads=2, head_dim=128, ffn=768, qk_norm=False,
                                   no_rope_interval=2), seed=9)
    prompt = np.random.default_rng(12).integers(0, spec.vocab, 96).astype(np.int32)
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=True, max_tokens=160)
    cpu = O.Model(spec, 160, kv_f16=True)
    got = dev.greedy(prompt, 32)
    ref, margins = cpu.greedy(prompt, 32)
    print("nope min margin", float(margins.min()), flush=True)
    assert np.array_equal(got, ref), (got, ref, margins)
    dev.close()
    cpu.close()


LONG = [
    ("qwen3-30b-a3b-q4_k_m", dict(layers=2, vocab=2048, hidden=512, heads=8, kv_heads=2,
                                  head_dim=128, experts=16, experts_used=4, expert_ffn=256)),
    ("gpt-oss-20b-mxfp4", dict(layers=2, vocab=2048, hidden=512, heads=8, kv_heads=2,
                               head_dim=64, experts=8, experts_used=2, expert_ffn=512,
                               window=160)),
]


@pytest.mark.parametrize("chunk", [1024, 100])
@pytest.mark.parametrize("name,over", LONG)
def test_tiny_greedy_long_context(ctx, name, over, chunk):
    # a context of several 128-key ranges (and a window across them): the
    # decode attention's ranges and their merge, replayed by the graph; the
    # prompt in one chunk, or in chunks of 100 rows (a chunk's rows start
    # inside a range and partway through the window)
    spec = models.Spec(models.tiny(name, **over), seed=57)
    prompt = np.random.default_rng(9).integers(0, spec.vocab, 300).astype(np.int32)
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=True, max_tokens=512)
    dev.chunk(chunk)
    cpu = O.Model(spec, 512, kv_f16=True, threads=16)
    got = dev.greedy(prompt, 24)
    ref, margins = cpu.greedy(prompt, 24)
    print(name, "min margin", float(margins.min()), flush=True)
    assert np.array_equal(got, ref), (got, ref, margins)
    dev.close()
    cpu.close()


@pytest.mark.parametrize("name,over", [TINY[2], TINY[3]])
def test_check_route_counts(ctx, name, over):
    """CheckRoute (model.qwen3.cuda.pas:288-300, :1207-1256): every decode
    step's on-device route of every MoE layer is read back and compared with
    TDecoderModel.Route on the host: the same ids, weights within 1e-6, the
    tokens those of a decode without the check (graphs on)."""
    spec = models.Spec(models.tiny(name, **over), seed=33)
    prompt = np.random.default_rng(5).integers(0, spec.vocab, 12).astype(np.int32)
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=64)
    want = dev.greedy(prompt, 10)
    dev.close()
    dev = H.Model(ctx, spec, mode=H.MODE_Q8, max_tokens=64)
    dev.check_route(True)
    got = dev.greedy(prompt, 10)
    checks, mismatches, max_diff = dev.route_stats()
    dev.close()
    assert np.array_equal(got, want)
    # the 10 decode steps after the prompt (Greedy feeds its last token too),
    # every layer routed
    assert checks == 10 * over["layers"], checks
    assert mismatches == 0 and max_diff <= 1e-6, (mismatches, max_diff)


def test_gptoss_f8f6f4_experts_greedy(ctx):
    """A gpt-oss-shaped model whose MXFP4 expert GEMMs (grouped items of the
    prompt) run on the scaled f8f6f4 matrix cores: the oracle's tokens."""
    import os
    name, over = TINY[3]
    spec = models.Spec(models.tiny(name, **over), seed=41)
    prompt = np.random.default_rng(9).integers(0, spec.vocab, 200).astype(np.int32)
    saved = os.environ.get("IHIP_GEMM_F8")
    os.environ["IHIP_GEMM_F8"] = "1"
    try:
        c = H.Context(0)
    finally:
        if saved is None:
            os.environ.pop("IHIP_GEMM_F8", None)
        else:
            os.environ["IHIP_GEMM_F8"] = saved
    dev = H.Model(c, spec, mode=H.MODE_Q8, max_tokens=256)
    got = dev.greedy(prompt, 16)
    dev.close()
    c.close()
    ref, margins = O.Model(spec, 256).greedy(prompt, 16)
    assert np.array_equal(got, ref), (got, ref, margins)
