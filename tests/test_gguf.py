"""The GGUF reader and the decoder description of a GGUF file, on the host (no
GPU): the reader against the reference's tiny file and damaged variants
(TTestInferGguf.ReaderReadsTinyFile / ReaderRefusesDamagedFiles,
tests/test.infer.gguf.pas:811-987), the llama.cpp model files and their
refusals (TTestInferQwen3, tests/test.infer.qwen3.pas:1485-1566, :5640-5660),
and the CPU oracle decoding them against the float32 logits transformers wrote
for the same weights (tests/golden/gguf/expected.npz)."""
import os
import struct

import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O

GG = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gguf")
EXP = np.load(os.path.join(GG, "expected.npz"))


# ------------------------------------------------- a tiny writer for variants
def u32(v):
    return struct.pack("<I", v & 0xFFFFFFFF)


def u64(v):
    return struct.pack("<Q", v & 0xFFFFFFFFFFFFFFFF)


def gstr(s):
    s = s if isinstance(s, bytes) else s.encode()
    return u64(len(s)) + s


def kv(key, t, payload):
    return gstr(key) + u32(t) + payload


def ti(name, dims, t, off):
    return gstr(name) + u32(len(dims)) + b"".join(u64(d) for d in dims) + u32(t) + u64(off)


def gfile(version, nt, nv, kvs, tis, data, align=32):
    b = b"GGUF" + u32(version) + u64(nt) + u64(nv) + kvs + tis
    b += b"\0" * (-len(b) % align)
    return b + data


DATA = b"\0" * (32 + 2 * 34)


def mini():
    """One string key, an F32 [4] and a Q8_0 [2, 32] tensor."""
    return gfile(3, 2, 1, kv("general.architecture", 8, gstr("x")),
                 ti("a", [4], 0, 0) + ti("b", [32, 2], 8, 32), DATA)


def refused(content, why=""):
    try:
        H.Gguf(content=content).close()
    except H.FormatError as e:
        return why in str(e)
    return False


# ------------------------------------------------------------------ reader
def test_reader_reads_tiny_file():
    with H.Gguf(os.path.join(GG, "model.gguf")) as g:
        assert g.str("general.architecture") == "bert"
        assert g.int("bert.block_count") == 2
        assert abs(g.float("bert.attention.layer_norm_epsilon") - 1e-5) < 1e-12
        assert g.bool("bert.attention.causal") is False
        assert g.bool("no.such.key", default=True) is True
        assert g.alignment == 32
        assert len(g.tensors()) == 5 + 16 * 2
        t = g.tensor("token_embd.weight")
        assert t["dtype"] == H.Q8_0 and t["shape"] == (64, 32) and t["bytes"] == 64 * 34
        t = g.tensor("position_embd.weight")
        assert t["dtype"] == H.F32 and t["shape"] == (38, 32)
        assert g.tensor("nope") is None
        with pytest.raises(H.FormatError, match="expected STRING"):
            g.str("bert.block_count")
        with pytest.raises(H.FormatError, match="is Q8_0, expected F32"):
            g.weight("token_embd.weight", H.F32, [64, 32])
        # tensors follow each other in file order, inside the file
        ts = g.tensors()
        for a, b in zip(ts, ts[1:]):
            assert a["data"] + a["bytes"] <= b["data"]


def test_reader_refuses_damaged_files():
    m = mini()
    assert not refused(m)
    with H.Gguf(content=m) as g:
        assert g.keys() == ["general.architecture"]
        assert [t["shape"] for t in g.tensors()] == [(4,), (2, 32)]
    cases = [
        (b"GGUX" + m[4:], "not a GGUF"),
        (gfile(2, 2, 1, kv("general.architecture", 8, gstr("x")),
               ti("a", [4], 0, 0) + ti("b", [32, 2], 8, 32), DATA), "version"),
        (gfile(3, 1 << 40, 1, b"", b"", b""), "cannot fit"),
        (gfile(3, 0, 1 << 62, b"", b"", b""), "cannot fit"),
        # key/value pairs
        (gfile(3, 0, 1, kv("k", 13, u32(0)), b"", b""), "unknown type"),
        (gfile(3, 0, 1, kv("k", 7, b"\x02"), b"", b""), "BOOL"),
        (gfile(3, 0, 1, kv("k", 8, gstr(b"a\0b")), b"", b""), "NUL"),
        (gfile(3, 0, 1, kv(b"k\0", 4, u32(1)), b"", b""), "NUL"),
        (gfile(3, 0, 1, kv("", 4, u32(1)), b"", b""), "empty key"),
        (gfile(3, 0, 2, kv("k", 4, u32(1)) + kv("k", 4, u32(2)), b"", b""), "twice"),
        (gfile(3, 0, 1, kv("k", 9, u32(9) + u64(1) + u32(4) + u64(1) + u32(0)), b"", b""),
         "nested"),
        (gfile(3, 0, 1, kv("k", 9, u32(4) + u64(1 << 60)), b"", b""), "more than the file"),
        (gfile(3, 0, 1, kv("k", 9, u32(8) + u64(1000)), b"", b""), "more than the file"),
        (gfile(3, 0, 1, kv("k", 8, u64(1 << 50)), b"", b""), "past the end"),
        (gfile(3, 0, 1, kv("k", 8, u64(-1)), b"", b""), "out of range"),
        (gfile(3, 0, 1, kv("general.alignment", 4, u32(24)), b"", b""), "power of two"),
        (gfile(3, 0, 1, kv("general.alignment", 4, u32(0)), b"", b""), "power of two"),
        (gfile(3, 0, 1, kv("general.alignment", 10, u64(32)), b"", b""), "UINT32"),
        # tensor infos
        (gfile(3, 1, 0, b"", ti("a", [4], 3, 0), DATA), "ggml type"),
        (gfile(3, 1, 0, b"", ti("a", [4], 2, 0), DATA), "blocks"),
        (gfile(3, 1, 0, b"", ti("a", [0], 0, 0), DATA), "dimension"),
        (gfile(3, 1, 0, b"", ti("a", [1, 1, 1, 1, 1], 0, 0), DATA), "dimensions"),
        (gfile(3, 1, 0, b"", ti("a", [], 0, 0), DATA), "dimensions"),
        (gfile(3, 1, 0, b"", ti("a", [48], 8, 0), DATA), "blocks"),
        (gfile(3, 1, 0, b"", ti("a", [1 << 40, 1 << 30], 0, 0), DATA), "exceeds"),
        (gfile(3, 1, 0, b"", ti("a", [4], 0, 4), DATA), "aligned"),
        (gfile(3, 2, 0, b"", ti("a", [4], 0, 0) + ti("a", [4], 0, 32), DATA), "twice"),
        (gfile(3, 2, 0, b"", ti("a", [16], 0, 0) + ti("b", [4], 0, 32), DATA), "expected"),
        (gfile(3, 2, 0, b"", ti("a", [4], 0, 0) + ti("b", [4], 0, 64), DATA), "expected"),
        (gfile(3, 2, 0, b"", ti("b", [4], 0, 32) + ti("a", [4], 0, 0), DATA), "expected"),
        (gfile(3, 1, 0, b"", ti("a", [64], 0, 0), DATA), "outside"),
        (gfile(3, 1, 0, b"", ti("a", [4], 0, 0), DATA), "unreferenced"),
    ]
    for content, why in cases:
        assert refused(content, why), why
    # the padding after the last tensor is fine
    assert not refused(gfile(3, 1, 0, b"", ti("a", [4], 0, 0), DATA[:31]))


def test_reader_truncations_and_flips():
    tiny = open(os.path.join(GG, "model.gguf"), "rb").read()
    assert not refused(tiny)
    # every truncation is refused, as a format error only
    for i in range(len(tiny)):
        if i < 4096 or i % 97 == 0:
            assert refused(tiny[:i]), i
    # flipped header bytes give a format error or a valid file, nothing else
    b = bytearray(tiny)
    for i in range(1, 8193):
        c = bytearray(b)
        j = (i * 7919) % 8192
        c[j] ^= 1 << (i & 7)
        try:
            H.Gguf(content=bytes(c)).close()
        except H.FormatError:
            pass


def test_reader_arrays_and_strings():
    kvs = (kv("f", 9, u32(6) + u64(3) + struct.pack("<3f", 1.5, -2.0, 3.25)) +
           kv("s", 9, u32(8) + u64(3) + gstr("ab") + gstr("") + gstr("xyz")) +
           kv("b", 9, u32(7) + u64(2) + b"\x01\x00") + kv("i", 11, u64(-5)) +
           kv("u", 10, u64(1 << 63)))
    g = H.Gguf(content=gfile(3, 0, 5, kvs, b"", b""))
    assert np.array_equal(g.array("f", H.GGUF_FLOAT32), np.float32([1.5, -2.0, 3.25]))
    assert g.strings("s") == ["ab", "", "xyz"]
    assert list(g.array("b", H.GGUF_BOOL)) == [1, 0]
    assert g.int("i") == -5
    with pytest.raises(H.FormatError, match="out of range"):
        g.int("u")  # a UINT64 above the int64 range
    with pytest.raises(H.FormatError, match="elements, expected 4"):
        g.array("f", H.GGUF_FLOAT32, 4)
    with pytest.raises(H.FormatError, match="array of FLOAT32, expected INT32"):
        g.array("f", H.GGUF_INT32)
    with pytest.raises(H.FormatError, match="no metadata"):
        g.float("nope")
    # a BOOL array with a 2 is refused at open
    assert refused(gfile(3, 0, 1, kv("b", 9, u32(7) + u64(2) + b"\x01\x02"), b"", b""), "BOOL")


# ------------------------------------------------------ the model files
def test_qwen3_settings_of_the_file():
    s = H.GgufSpec(os.path.join(GG, "qwen3", "q8_0.gguf"))
    d = s.struct
    # tiny-qwen3/config.json
    assert (d.vocab, d.hidden, d.layers, d.heads, d.kv_heads, d.head_dim, d.ffn) == \
        (96, 64, 2, 4, 2, 32, 160)
    assert d.max_positions == 512 and d.rope_theta == 1e6 and abs(d.rms_eps - 1e-6) < 1e-12
    assert d.head.data is None  # no output.weight: tied
    assert d.embed.dtype == H.Q8_0 and s.layers[0].q.dtype == H.Q8_0
    assert s.layers[0].q_norm.data and s.layers[0].moe == 0
    s4 = H.GgufSpec(os.path.join(GG, "qwen3", "q4_0.gguf"))
    assert s4.layers[1].down.dtype == H.Q4_0 and s4.struct.embed.dtype == H.Q8_0
    su = H.GgufSpec(os.path.join(GG, "qwen3", "untied-f16.gguf"))
    assert su.struct.head.data and su.struct.head.dtype == H.F16


def test_qwen2_settings_of_the_file():
    # tiny-qwen2 as llama.cpp writes a qwen2 file (TTestInferQwen3.
    # TinyQwen2MatchesReference, tests/test.infer.qwen3.pas:2532-2606): no
    # attention.key_length, so head_dim = hidden / heads = 16; F32 biases on
    # q, k and v, no head norm
    s = H.GgufSpec(os.path.join(GG, "qwen2", "q8_0.gguf"))
    d = s.struct
    assert (d.vocab, d.hidden, d.layers, d.heads, d.kv_heads, d.head_dim, d.ffn) == \
        (96, 64, 2, 4, 2, 16, 160)
    assert d.head.data is None  # tied
    for L in s.layers:
        assert L.q_bias.data and L.k_bias.data and L.v_bias.data and not L.o_bias.data
        assert not L.q_norm.data and not L.k_norm.data and L.q.dtype == H.Q8_0


def test_qwen3moe_and_gptoss_settings():
    s = H.GgufSpec(os.path.join(GG, "qwen3moe", "q8_0.gguf"))
    d = s.struct
    assert (d.experts, d.experts_used, d.expert_ffn, d.norm_topk) == (8, 2, 64, 1)
    assert [L.moe for L in s.layers] == [1, 0, 1]  # mlp_only_layers [1]
    assert s.layers[0].exp_gate.dtype == H.Q8_0 and s.layers[0].router.dtype == H.F32
    g = H.GgufSpec(os.path.join(GG, "gpt-oss", "bf16.gguf"))
    d = g.struct
    assert (d.experts, d.experts_used, d.expert_ffn, d.head_dim) == (8, 3, 64, 24)
    assert (d.swiglu_alpha, d.swiglu_limit) == (pytest.approx(1.702), 7.0)
    assert (d.rope_factor, d.rope_original, d.rope_beta_fast, d.rope_beta_slow) == \
        (32.0, 4096, 32.0, 1.0)
    assert [L.window for L in g.layers] == [5, 0, 5]  # the even layers slide
    assert all(L.moe and L.sinks.data and L.exp_down_bias.data for L in g.layers)
    assert g.layers[0].exp_up.dtype == H.MXFP4 and g.layers[0].q.dtype == H.BF16
    b = H.GgufSpec(os.path.join(GG, "gpt-oss", "betas.gguf")).struct
    assert (b.rope_beta_fast, b.rope_beta_slow) == (16.0, 2.0)


@pytest.mark.parametrize("arch,name,why", [
    ("qwen3", "bad-arch", "architecture"), ("qwen3", "bad-rope", "rope scaling"),
    ("qwen3", "bad-extra", "understood"), ("qwen3", "bad-missing", "no tensor"),
    ("qwen3", "bad-scale", "no finite number"), ("qwen3", "bad-shape", "shaped"),
    ("qwen3", "bad-ropedim", "RoPE over"), ("qwen3", "bad-embscale", "no finite number"),
    ("qwen3moe", "bad-experts", "shaped"),
    ("gpt-oss", "bad-arch", "architecture"), ("gpt-oss", "bad-rope", "rope scaling"),
    ("gpt-oss", "bad-yarn", "attention factor"), ("gpt-oss", "bad-tied", "tied embeddings"),
    ("gpt-oss", "bad-missing", "attn_sinks"), ("gpt-oss", "bad-extra", "understood"),
    ("gpt-oss", "bad-scale", "beyond the range"), ("qwen2", "bad-nobias", "attn_k.bias")])
def test_model_refuses_damaged_files(arch, name, why):
    with pytest.raises(H.FormatError, match=why):
        H.GgufSpec(os.path.join(GG, "bad", arch, name + ".gguf"))


def test_reader_accepts_every_damaged_model_file():
    # the damage is in the model, not in the file format
    for arch in ("qwen3", "qwen3moe", "gpt-oss", "qwen2"):
        for n in os.listdir(os.path.join(GG, "bad", arch)):
            H.Gguf(os.path.join(GG, "bad", arch, n)).close()


# ------------------------------------- the oracle against transformers
def cos(a, b):
    a, b = a.ravel().astype(np.float64), b.ravel().astype(np.float64)
    return float(a @ b / np.linalg.norm(a) / np.linalg.norm(b))


def expected(tag):
    n = sum(1 for k in EXP.files if k.startswith(tag + "/") and k.endswith(".ids"))
    return [{f: EXP[f"{tag}/case{k}.{f}"] for f in ("ids", "logits", "greedy", "greedy_margin")
             if f"{tag}/case{k}.{f}" in EXP.files} for k in range(n)]


@pytest.mark.parametrize("file,tag,mode,min_cos", [
    ("qwen3/q8_0.gguf", "qwen3", "q8", 0.999),
    ("qwen3/q8_0.gguf", "qwen3", "f32", 0.999),
    ("qwen3moe/q8_0.gguf", "qwen3moe", "q8", 0.999),
    ("qwen3moe/q8_0.gguf", "qwen3moe", "f32", 0.999),
    ("qwen2/q8_0.gguf", "qwen2", "q8", 0.999),
    ("qwen2/q8_0.gguf", "qwen2", "f32", 0.999)])
def test_oracle_q8_0_file_vs_transformers(file, tag, mode, min_cos):
    # Q8_0 weights against the float32 logits of the BF16 checkpoint: within
    # the Q8_0 error (the reference's own bound, test.infer.qwen3.pas:1527)
    s = H.GgufSpec(os.path.join(GG, file))
    for c in expected(tag):
        m = O.Model(s, 64, f32=(mode == "f32"))
        lg = m.forward(c["ids"], all_logits=True)
        assert cos(lg, c["logits"]) > min_cos
        assert np.abs(lg - c["logits"]).max() < 0.1
        m.close()


def test_oracle_f16_file_vs_transformers():
    # F16 matrices widen exactly: the float32 logits of transformers to ~1e-6
    s = H.GgufSpec(os.path.join(GG, "qwen3", "untied-f16.gguf"))
    for c in expected("qwen3-untied"):
        for f32 in (False, True):
            lg = O.Model(s, 64, f32=f32).forward(c["ids"], all_logits=True)
            assert np.abs(lg - c["logits"]).max() < 1e-5


def test_oracle_gptoss_file_vs_transformers():
    # bf16.gguf holds the checkpoint's values; llama.cpp fixes the SwiGLU
    # limit at 7 where the checkpoint has 0.8, so with 0.8 set the F32
    # arithmetic gives transformers' logits (YaRN, sinks, windows, biases,
    # MXFP4 experts, head_dim 24) and its greedy tokens
    s = H.GgufSpec(os.path.join(GG, "gpt-oss", "bf16.gguf"))
    s.struct.swiglu_limit = 0.8
    for c in expected("gpt-oss"):
        m = O.Model(s, 80, f32=True)
        lg = m.forward(c["ids"], all_logits=True)
        assert np.abs(lg - c["logits"]).max() < 1e-5
        ids, _ = O.Model(s, 80, f32=True).greedy(c["ids"], len(c["greedy"]))
        assert np.array_equal(ids, c["greedy"])
