"""Copy the reference's GGUF test files and the transformers expectations the
reference's tests compare them with into tests/golden/gguf/ (data only).

Sources, under tests/data/infer-ref/ of the reference (written by llama.cpp's
converter and ggml's reference quantizers, and by transformers in float32):
- tiny-gguf/model.gguf: the reader fixture of TTestInferGguf.ReaderReadsTinyFile
  (tests/test.infer.gguf.pas:811-857);
- tiny-qwen3-gguf/{q8_0,q4_0,untied-f16,bad-*}.gguf, tiny-qwen3moe/gguf/*.gguf,
  tiny-gpt-oss/gguf/*.gguf: the model files of TTestInferQwen3
  (tests/test.infer.qwen3.pas:1485-1566, :5600-5660) and the device tests
  (tests/test.infer.cuda.pas:1560-1640, :1950-2010);
- tiny-qwen35/gguf/{bf16,q8_0,text-bf16,text-q8_0,bad-*}.gguf: the qwen35
  files of TTestInferQwen35 (tests/test.infer.qwen35.pas) and the device
  tests of the DeltaNet (tests/test.infer.cuda.pas);
- tiny-gemma4/gguf/{bf16,q8_0,dense-bf16,dense-q8_0,rope44,bad-*}.gguf: the
  gemma4 files of TTestInferGemma4 (tests/test.infer.gemma4.pas);
- tiny-qwen2/gguf/{q8_0,bad-nobias}.gguf: the qwen2 (Qwen2.5) files of
  TTestInferQwen3's Qwen2 cases (the decoder with q/k/v biases and no head
  norms);
- the case ids, logits, greedy tokens and margins of tiny-qwen3,
  tiny-qwen3/untied, tiny-qwen3moe, tiny-gpt-oss/mxfp4, tiny-qwen35 and
  tiny-qwen35/text (with the one-token-at-a-time logits and the first layer's
  mixer output of the last two), tiny-gemma4, tiny-gemma4/dense and tiny-qwen2
  (tensors.bin, described by manifest.json),
  gathered into expected.npz.

Every file is checked against the sha256 its manifest records before it is
copied. The damaged files go to gguf/bad/ (CPU tests only). Run from the
repository root: python tests/golden/copy_gguf_fixtures.py [reference root]
"""
import hashlib
import json
import os
import shutil
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "gguf")


def sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def copy_dir(src, names, dst, manifest_files):
    os.makedirs(dst, exist_ok=True)
    for n in names:
        p = os.path.join(src, n)
        want = manifest_files.get(n)
        if want and sha(p) != want:
            raise SystemExit(f"{p}: sha256 differs from its manifest")
        shutil.copyfile(p, os.path.join(dst, n))


def cases(folder):
    m = json.load(open(os.path.join(folder, "manifest.json")))
    blob = open(os.path.join(folder, "tensors.bin"), "rb").read()
    if sha(os.path.join(folder, "tensors.bin")) != m["blob"]["sha256"]:
        raise SystemExit(f"{folder}: tensors.bin sha256 differs from its manifest")
    out = {}
    for t in m["tensors"]:
        name = t["name"]
        if not name.startswith("case") or name.split(".", 1)[1] not in (
                "ids", "logits", "greedy", "greedy_margin", "logits_steps", "layer00_attn"):
            continue
        dt = {"f32": np.float32, "i32": np.int32}[t["dtype"]]
        a = np.frombuffer(blob[t["offset"]:t["offset"] + t["bytes"]], dt).reshape(t["shape"])
        out[name] = a.copy()
    return out


def main(ref):
    root = os.path.join(ref, "tests", "data", "infer-ref")
    os.makedirs(OUT, exist_ok=True)
    # the reader fixture
    copy_dir(os.path.join(root, "tiny-gguf"), ["model.gguf"], OUT, {})
    sets = [("tiny-qwen3-gguf", "qwen3"), (os.path.join("tiny-qwen3moe", "gguf"), "qwen3moe"),
            (os.path.join("tiny-gpt-oss", "gguf"), "gpt-oss"), (os.path.join("tiny-qwen35", "gguf"), "qwen35"),
            (os.path.join("tiny-gemma4", "gguf"), "gemma4"), (os.path.join("tiny-qwen2", "gguf"), "qwen2")]
    for folder, tag in sets:
        src = os.path.join(root, folder)
        files = json.load(open(os.path.join(src, "manifest.json"))).get("files", {})
        good = [n for n in sorted(os.listdir(src)) if n.endswith(".gguf") and not n.startswith(
            ("bad-", "tok-", "tokenizer"))]
        bad = [n for n in sorted(os.listdir(src)) if n.startswith("bad-") and n.endswith(".gguf")
               and not n.startswith("bad-tokenizer")]
        copy_dir(src, good, os.path.join(OUT, tag), files)
        copy_dir(src, bad, os.path.join(OUT, "bad", tag), files)
    expected = {}
    for folder, tag in [("tiny-qwen3", "qwen3"), (os.path.join("tiny-qwen3", "untied"), "qwen3-untied"),
                        ("tiny-qwen3moe", "qwen3moe"), (os.path.join("tiny-gpt-oss", "mxfp4"), "gpt-oss"),
                        ("tiny-qwen35", "qwen35"), (os.path.join("tiny-qwen35", "text"), "qwen35-text"),
                        ("tiny-gemma4", "gemma4"), (os.path.join("tiny-gemma4", "dense"), "gemma4-dense"),
                        ("tiny-qwen2", "qwen2")]:
        for k, v in cases(os.path.join(root, folder)).items():
            expected[f"{tag}/{k}"] = v
    np.savez_compressed(os.path.join(OUT, "expected.npz"), **expected)
    print("wrote", OUT)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
