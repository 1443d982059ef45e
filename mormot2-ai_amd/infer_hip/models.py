"""Seeded synthetic decoders of the BASELINE configurations (random weights of
the real architectures: there is no network for checkpoints), described by the
C-ABI's ihip_model_desc so the HIP device and the CPU oracle read the very
same host bytes.

Shapes: Qwen3-0.6B (decoder.pas / model.qwen3.pas), Qwen3-30B-A3B (MoE with
128 experts, top-8 renormalised), gpt-oss-20b (model.gptoss.pas: biases,
sinks, alternating 128-token windows, YaRN, clamped SwiGLU, MXFP4 experts).
"""
import ctypes as C

import numpy as np

from . import (BF16, F32, MXFP4, Q4_K, Q6_K, Q8_0, LayerDesc, ModelDesc, Tensor, row_bytes,
               synth_normal)

CONFIGS = {
    # Qwen3-0.6B, Q8_0 (ties away, as GGUF writers quantize)
    "qwen3-0.6b-q8_0": dict(vocab=151936, hidden=1024, layers=28, heads=16, kv_heads=8,
                            head_dim=128, ffn=3072, rope_theta=1e6, rms_eps=1e-6, qk_norm=True,
                            tied=True, quant="q8_0"),
    # the same shape, Q4_K_M mixing
    "qwen3-0.6b-q4_k_m": dict(vocab=151936, hidden=1024, layers=28, heads=16, kv_heads=8,
                              head_dim=128, ffn=3072, rope_theta=1e6, rms_eps=1e-6, qk_norm=True,
                              tied=True, quant="q4_k_m"),
    # Qwen3-30B-A3B, Q4_K_M
    "qwen3-30b-a3b-q4_k_m": dict(vocab=151936, hidden=2048, layers=48, heads=32, kv_heads=4,
                                 head_dim=128, experts=128, experts_used=8, expert_ffn=768,
                                 rope_theta=1e6, rms_eps=1e-6, qk_norm=True, tied=False,
                                 quant="q4_k_m", moe=True),
    # gpt-oss-20b, MXFP4 experts, bf16 attention/router/head
    "gpt-oss-20b-mxfp4": dict(vocab=201088, hidden=2880, layers=24, heads=64, kv_heads=8,
                              head_dim=64, experts=32, experts_used=4, expert_ffn=2880,
                              rope_theta=150000.0, rms_eps=1e-5, qk_norm=False, tied=False,
                              quant="gptoss", moe=True, window=128, yarn=(32.0, 4096, 32.0, 1.0),
                              swiglu=(1.702, 7.0), biases=True, sinks=True),
}


def tiny(name, layers=2, vocab=1024, **over):
    """A small model of the same family (tests): fewer layers, a small vocabulary."""
    cfg = dict(CONFIGS[name])
    cfg.update(layers=layers, vocab=vocab)
    cfg.update(over)
    return cfg


class Spec:
    """Host tensors + the ModelDesc that points at them."""

    def __init__(self, cfg, seed=1, sigma=0.02):
        self.cfg = cfg
        self.keep = []
        self._seed = seed
        c = cfg
        H, hd = c["hidden"], c["head_dim"]
        qw, kvw = c["heads"] * hd, c["kv_heads"] * hd
        moe = c.get("moe", False)
        E, K, FI = c.get("experts", 0), c.get("experts_used", 0), c.get("expert_ffn", 0)
        F = c.get("ffn", 0)
        q = c["quant"]
        d = ModelDesc()
        d.vocab, d.hidden, d.layers = c["vocab"], H, c["layers"]
        d.heads, d.kv_heads, d.head_dim = c["heads"], c["kv_heads"], hd
        d.ffn, d.experts, d.experts_used, d.expert_ffn = F, E, K, FI
        d.norm_topk = 1 if moe else 0
        d.max_positions = 1 << 20
        d.rms_eps = c["rms_eps"]
        a, lim = c.get("swiglu", (1.0, 0.0))
        d.swiglu_alpha, d.swiglu_limit = a, lim
        d.rope_theta = c["rope_theta"]
        if "yarn" in c:
            d.rope_factor, d.rope_original, d.rope_beta_fast, d.rope_beta_slow = c["yarn"]
            d.rope_truncate = 0
        # token embedding and head
        if q == "q8_0":
            emb_t, head_t = Q8_0, Q8_0
        elif q == "q4_k_m":
            emb_t, head_t = (Q6_K, Q6_K) if c["tied"] else (Q4_K, Q6_K)
        else:
            emb_t, head_t = BF16, BF16
        d.embed = self.mat(emb_t, c["vocab"], H, sigma)
        d.head = Tensor() if c["tied"] else self.mat(head_t, c["vocab"], H, sigma)
        d.final_norm = self.ones(H)
        layers = (LayerDesc * c["layers"])()
        for li in range(c["layers"]):
            L = layers[li]
            if q == "q8_0":
                at = [Q8_0] * 4
                ft = [Q8_0] * 3
            elif q == "q4_k_m":
                at = [Q4_K, Q4_K, Q6_K, Q4_K]
                ft = [Q4_K, Q4_K, Q6_K if li % 2 == 0 else Q4_K]
            else:
                at = [BF16] * 4
                ft = [MXFP4] * 3
            L.input_norm = self.ones(H)
            L.post_norm = self.ones(H)
            L.q = self.mat(at[0], qw, H, sigma)
            L.k = self.mat(at[1], kvw, H, sigma)
            L.v = self.mat(at[2], kvw, H, sigma)
            L.o = self.mat(at[3], H, qw, sigma)
            if c.get("qk_norm"):
                L.q_norm = self.ones(hd)
                L.k_norm = self.ones(hd)
            if c.get("biases"):
                L.q_bias = self.vec(qw, sigma)
                L.k_bias = self.vec(kvw, sigma)
                L.v_bias = self.vec(kvw, sigma)
                L.o_bias = self.vec(H, sigma)
            if c.get("sinks"):
                L.sinks = self.vec(c["heads"], 1.0)
            if c.get("window") and li % 2 == 0:
                L.window = c["window"]
            if moe:
                L.moe = 1
                rt = BF16 if q == "gptoss" else F32
                L.router = self.mat(rt, E, H, sigma)
                if c.get("biases"):
                    L.router_bias = self.vec(E, sigma)
                    L.exp_gate_bias = self.vec(E * FI, sigma)
                    L.exp_up_bias = self.vec(E * FI, sigma)
                    L.exp_down_bias = self.vec(E * H, sigma)
                L.exp_gate = self.mat(ft[0], E * FI, H, sigma)
                L.exp_up = self.mat(ft[1], E * FI, H, sigma)
                L.exp_down = self.mat(ft[2], E * H, FI, sigma)
            else:
                L.gate = self.mat(ft[0], F, H, sigma)
                L.up = self.mat(ft[1], F, H, sigma)
                L.down = self.mat(ft[2], H, F, sigma)
        self.layers = layers
        d.layer = C.cast(layers, C.POINTER(LayerDesc))
        self.struct = d
        self.vocab = c["vocab"]

    def _next(self):
        self._seed += 1
        return self._seed * 7919 + 13

    def mat(self, dtype, rows, cols, sigma):
        a = synth_normal(dtype, rows, cols, self._next(), sigma)
        self.keep.append(a)
        return Tensor(a.ctypes.data, dtype, 0)

    def vec(self, n, sigma):
        a = (np.random.default_rng(self._next()).standard_normal(n) * sigma).astype(np.float32)
        self.keep.append(a)
        return Tensor(a.ctypes.data, F32, 0)

    def ones(self, n):
        a = np.ones(n, np.float32)
        self.keep.append(a)
        return Tensor(a.ctypes.data, F32, 0)

    def weight_bytes_per_token(self):
        """Bytes of the weights one decode step reads (all dense matrices,
        the k experts of each MoE layer, the head; norms and biases aside)."""
        c = self.cfg
        H, hd = c["hidden"], c["head_dim"]
        total = 0
        d = self.struct
        for li in range(c["layers"]):
            L = self.layers[li]
            for name, rows, cols in (("q", c["heads"] * hd, H), ("k", c["kv_heads"] * hd, H),
                                     ("v", c["kv_heads"] * hd, H), ("o", H, c["heads"] * hd)):
                total += rows * row_bytes(getattr(L, name).dtype, cols)
            if L.moe:
                E, K, FI = c["experts"], c["experts_used"], c["expert_ffn"]
                total += E * row_bytes(L.router.dtype, H)
                total += K * FI * (row_bytes(L.exp_gate.dtype, H) + row_bytes(L.exp_up.dtype, H))
                total += K * H * row_bytes(L.exp_down.dtype, FI)
            else:
                F = c["ffn"]
                total += F * (row_bytes(L.gate.dtype, H) + row_bytes(L.up.dtype, H))
                total += H * row_bytes(L.down.dtype, F)
        head = d.head if d.head.data else d.embed
        total += c["vocab"] * row_bytes(head.dtype, H)
        return total
