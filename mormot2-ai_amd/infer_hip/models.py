"""Seeded synthetic decoders of the BASELINE configurations (random weights of
the real architectures: there is no network for checkpoints), described by the
C-ABI's ihip_model_desc so the HIP device and the CPU oracle read the very
same host bytes.

Shapes: Qwen3-0.6B (decoder.pas / model.qwen3.pas), Qwen3-30B-A3B (MoE with
128 experts, top-8 renormalised), gpt-oss-20b (model.gptoss.pas: biases,
sinks, alternating 128-token windows, YaRN, clamped SwiGLU, MXFP4 experts);
beyond the BASELINE configurations, Qwen3.5-0.8B (model.qwen35.pas: Gated
DeltaNet layers, every fourth a gated full attention) and Gemma-4-26B-A4B
(model.gemma4.pas: five sliding layers of heads of 256 to one full layer of
heads of 512 with K=V, the dense block beside 128 experts, softcap 30), with
the settings of the reference's own reference manifests
(tests/data/infer-ref/qwen35-0.8b, gemma4-26b-a4b).
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
    # Qwen3.5-0.8B (no BASELINE config names it): 24 layers, every fourth a
    # gated full attention of 8 heads of 256 (a quarter rotating), the others
    # Gated DeltaNet with 16 key and 16 value heads of 128, a convolution of 4
    "qwen35-0.8b-q8_0": dict(family="qwen35", vocab=248320, hidden=1024, layers=24, heads=8,
                             kv_heads=2, head_dim=256, ffn=3584, rope_theta=1e7, rms_eps=1e-6,
                             rope_dims=64, lin_key_heads=16, lin_value_heads=16, lin_key_dim=128,
                             lin_value_dim=128, lin_conv=4, interval=4, tied=True, quant="q8_0"),
    # Gemma-4-26B-A4B (no BASELINE config names it): 30 layers, five sliding
    # (window 1024, 8 KV heads of 256) to one full (2 KV heads of 512, K=V, 64
    # of 256 pairs of the second set rotating), a dense GeGLU of 2112 beside
    # 128 experts of 704 (top 8), softcap 30
    "gemma4-26b-a4b-q8_0": dict(family="gemma4", vocab=262144, hidden=2816, layers=30, heads=16,
                                kv_heads=8, head_dim=256, full_head_dim=512, full_kv_heads=2,
                                window=1024, pattern=6, ffn=2112, experts=128, experts_used=8,
                                expert_ffn=704, rope_theta=1e4, rope2_theta=1e6, rope2_pairs=64,
                                rms_eps=1e-6, softcap=30.0, tied=True, quant="q8_0"),
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
        if c.get("family") in ("qwen35", "gemma4"):
            getattr(self, "_" + c["family"])(c, sigma)
            return
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
            # SmolLM3's NoPE layers: every no_rope_interval-th layer without
            # rotary positions (no_rope_layer_interval, model.qwen3.pas:28-33)
            if c.get("no_rope_interval") and (li + 1) % c["no_rope_interval"] == 0:
                L.no_rope = 1
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

    def _qwen35(self, c, sigma):
        """TQwen35Model's layout (model.qwen35.pas:534-640) in Q8_0: DeltaNet
        layers, every interval-th a gated attention; norms 1 + weight folded
        (ones here), -exp(A_log) stored as GGUF does."""
        H, hd, F = c["hidden"], c["head_dim"], c["ffn"]
        qw, kvw = c["heads"] * hd, c["kv_heads"] * hd
        kh, vh, dk, dv, kw = (c["lin_key_heads"], c["lin_value_heads"], c["lin_key_dim"],
                              c["lin_value_dim"], c["lin_conv"])
        vd, cd = vh * dv, 2 * kh * dk + vh * dv
        d = ModelDesc()
        d.vocab, d.hidden, d.layers = c["vocab"], H, c["layers"]
        d.heads, d.kv_heads, d.head_dim, d.ffn = c["heads"], c["kv_heads"], hd, F
        d.max_positions = 1 << 20
        d.rms_eps, d.rope_theta, d.rope_dims = c["rms_eps"], c["rope_theta"], c["rope_dims"]
        d.swiglu_alpha = 1.0
        d.lin_key_heads, d.lin_value_heads, d.lin_key_dim, d.lin_value_dim = kh, vh, dk, dv
        d.lin_conv, d.lin_tiled = kw, int(vh != kh)
        d.embed = self.mat(Q8_0, c["vocab"], H, sigma)
        d.final_norm = self.ones(H)
        layers = (LayerDesc * c["layers"])()
        rng = np.random.default_rng(self._next())
        for li in range(c["layers"]):
            L = layers[li]
            L.input_norm, L.post_norm = self.ones(H), self.ones(H)
            L.gate, L.up = self.mat(Q8_0, F, H, sigma), self.mat(Q8_0, F, H, sigma)
            L.down = self.mat(Q8_0, H, F, sigma)
            if (li + 1) % c["interval"]:
                L.mixer = 1
                L.lin_qkv = self.mat(Q8_0, cd, H, sigma)
                L.lin_z = self.mat(Q8_0, vd, H, sigma)
                L.lin_b, L.lin_a = self.mat(Q8_0, vh, H, sigma), self.mat(Q8_0, vh, H, sigma)
                L.lin_out = self.mat(Q8_0, H, vd, sigma)
                L.lin_conv = self.arr((rng.standard_normal(cd * kw) * 0.3).astype(np.float32))
                L.lin_dt_bias = self.arr((rng.standard_normal(vh) * 0.5).astype(np.float32))
                L.lin_neg_a = self.arr(-np.exp(rng.standard_normal(vh) * 0.5).astype(np.float32))
                L.lin_norm = self.ones(dv)
            else:
                L.output_gate = 1
                L.q = self.mat(Q8_0, 2 * qw, H, sigma)
                L.k, L.v = self.mat(Q8_0, kvw, H, sigma), self.mat(Q8_0, kvw, H, sigma)
                L.o = self.mat(Q8_0, H, qw, sigma)
                L.q_norm, L.k_norm = self.ones(hd), self.ones(hd)
        self.layers = layers
        d.layer = C.cast(layers, C.POINTER(LayerDesc))
        self.struct = d
        self.vocab = c["vocab"]

    def _gemma4(self, c, sigma):
        """TGemma4Model's layout (model.gemma4.pas:791-860) in Q8_0: sliding
        and full layers of their own heads, K=V in the full ones, the dense
        block beside the experts (gate and up of an expert in one tensor),
        the router norm folded with hidden^-0.5, layer scalars."""
        H, F = c["hidden"], c["ffn"]
        E, K, FI = c["experts"], c["experts_used"], c["expert_ffn"]
        d = ModelDesc()
        d.vocab, d.hidden, d.layers = c["vocab"], H, c["layers"]
        d.heads, d.kv_heads, d.head_dim, d.ffn = c["heads"], c["kv_heads"], c["head_dim"], F
        d.experts, d.experts_used, d.expert_ffn, d.norm_topk = E, K, FI, 1
        d.max_positions = 1 << 20
        d.rms_eps, d.rope_theta = c["rms_eps"], c["rope_theta"]
        d.rope2_theta, d.rope2_pairs = c["rope2_theta"], c["rope2_pairs"]
        d.swiglu_alpha = 1.0
        d.activation, d.value_norm, d.attention_scale = 1, 1, 1.0
        d.embed_scale = float(np.float32(np.sqrt(H)))
        d.logit_softcap = c["softcap"]
        d.embed = self.mat(Q8_0, c["vocab"], H, sigma)
        d.final_norm = self.ones(H)
        layers = (LayerDesc * c["layers"])()
        rng = np.random.default_rng(self._next())
        root = np.float32(1 / np.sqrt(H))
        for li in range(c["layers"]):
            L = layers[li]
            full = (li + 1) % c["pattern"] == 0
            hd = c["full_head_dim"] if full else c["head_dim"]
            kvh = c["full_kv_heads"] if full else c["kv_heads"]
            qw, kvw = c["heads"] * hd, kvh * hd
            if full:
                L.head_dim, L.kv_heads, L.k_is_v, L.rope_set = hd, kvh, 1, 1
            else:
                L.kv_heads, L.window = kvh, c["window"]
            L.q, L.k = self.mat(Q8_0, qw, H, sigma), self.mat(Q8_0, kvw, H, sigma)
            if not full:
                L.v = self.mat(Q8_0, kvw, H, sigma)
            L.o = self.mat(Q8_0, H, qw, sigma)
            L.q_norm, L.k_norm = self.ones(hd), self.ones(hd)
            for n in ("input_norm", "attn_out_norm", "post_norm", "ffn_out_norm",
                      "dense_out_norm", "moe_in_norm", "moe_out_norm"):
                setattr(L, n, self.ones(H))
            L.scalar = self.arr(rng.uniform(0.6, 1.4, 1).astype(np.float32))
            L.gate, L.up = self.mat(Q8_0, F, H, sigma), self.mat(Q8_0, F, H, sigma)
            L.down = self.mat(Q8_0, H, F, sigma)
            L.moe = 2
            L.router = self.mat(F32, E, H, sigma)
            L.router_norm = self.arr(np.full(H, root, np.float32))
            L.expert_scale = self.arr(rng.uniform(0.5, 1.5, E).astype(np.float32))
            L.exp_gate_up = 1
            L.exp_gate = self.mat(Q8_0, E * 2 * FI, H, sigma)
            L.exp_down = self.mat(Q8_0, E * H, FI, sigma)
        self.layers = layers
        d.layer = C.cast(layers, C.POINTER(LayerDesc))
        self.struct = d
        self.vocab = c["vocab"]

    def arr(self, a):
        self.keep.append(a)
        return Tensor(a.ctypes.data, F32, 0)

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
        H = c["hidden"]
        total = 0
        d = self.struct
        for li in range(c["layers"]):
            L = self.layers[li]
            hd = L.head_dim or c["head_dim"]
            kvh = L.kv_heads or c["kv_heads"]
            if L.mixer == 1:
                vd = d.lin_value_heads * d.lin_value_dim
                cd = 2 * d.lin_key_heads * d.lin_key_dim + vd
                for name, rows, cols in (("lin_qkv", cd, H), ("lin_z", vd, H),
                                         ("lin_b", d.lin_value_heads, H),
                                         ("lin_a", d.lin_value_heads, H), ("lin_out", H, vd)):
                    total += rows * row_bytes(getattr(L, name).dtype, cols)
            else:
                qrows = (2 if L.output_gate else 1) * c["heads"] * hd
                for name, rows, cols in (("q", qrows, H), ("k", kvh * hd, H),
                                         ("v", kvh * hd, H), ("o", H, c["heads"] * hd)):
                    if getattr(L, name).data:
                        total += rows * row_bytes(getattr(L, name).dtype, cols)
            if L.moe != 1:
                F = c["ffn"]
                total += F * (row_bytes(L.gate.dtype, H) + row_bytes(L.up.dtype, H))
                total += H * row_bytes(L.down.dtype, F)
            if L.moe == 2:
                E, K, FI = c["experts"], c["experts_used"], c["expert_ffn"]
                total += E * row_bytes(L.router.dtype, H)
                total += K * FI * 2 * row_bytes(L.exp_gate.dtype, H)
                total += K * H * row_bytes(L.exp_down.dtype, FI)
            if L.moe == 1:
                E, K, FI = c["experts"], c["experts_used"], c["expert_ffn"]
                total += E * row_bytes(L.router.dtype, H)
                total += K * FI * (row_bytes(L.exp_gate.dtype, H) + row_bytes(L.exp_up.dtype, H))
                total += K * H * row_bytes(L.exp_down.dtype, FI)
        head = d.head if d.head.data else d.embed
        total += c["vocab"] * row_bytes(head.dtype, H)
        return total
