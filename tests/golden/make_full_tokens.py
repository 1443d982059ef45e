"""Write the CPU oracle's greedy tokens at the benchmark's own workloads into
tests/golden/full_tokens/<config>.json (data: the device test compares with
them on the GPU box, where the oracle would need most of an hour).

For each configuration: the seeded synthetic weights of infer_hip.models
(seed 1), the prompt of the benchmark's length drawn from
numpy.random.default_rng(2024), the half-float KV cache of the device
default, then TDecoderModel.Greedy on the oracle one Forward per step
(decoder.pas Greedy; the reference's device test at full shape is
tests/test.infer.cuda.pas:2100-2232). Each step records the top-1/top-2
margin of the CPU logits and, for MoE models, the smallest k-th/(k+1)-th
router logit gap of the rows routed in it, so the device test can tell a
real mismatch from a near tie. The prompt's last-row logits of the 16 best
ids are kept too. With --tape, the oracle's expert choice of every routed
row (TDecoderRouteTape in record mode) goes to <config>.routes.npz: the
device test hands it to the device as the reference's own device test does,
so a near tie of the router (a k-th/(k+1)-th gap of a few ulps among the
tens of thousands of prompt routes) cannot send one row to other experts.

The synthetic weights depend only on the seed (ihip_synth_normal, checked by
tests/test_gpu_model.py::test_synth_deterministic_any_thread_count), so the
GPU box rebuilds the very bytes used here.

Run from the repository root:
  python tests/golden/make_full_tokens.py [config ...] [--threads N]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "mormot2-ai_amd"), os.path.join(ROOT, "tests")]

OUT = os.path.join(HERE, "full_tokens")
# the benchmark's prompt of each configuration ([2], [3], [4])
WORKLOADS = {"qwen3-30b-a3b-q4_k_m": 1024, "gpt-oss-20b-mxfp4": 2048,
             "qwen3-0.6b-q4_k_m": 512, "qwen3-0.6b-q8_0": 32}
STEPS = 64
SEED, PROMPT_SEED = 1, 2024
# the device's prompt chunk (ihip_model_chunk default); the oracle's results
# do not depend on how the prompt is cut, the order of its routed rows does
CHUNK = 1024


def prompt_of(vocab, n):
    return np.random.default_rng(PROMPT_SEED).integers(0, vocab, n).astype(np.int32)


def generate(name, threads, tape):
    import oracle_lib as O
    from infer_hip import models

    n = WORKLOADS[name]
    t0 = time.time()
    spec = models.Spec(models.CONFIGS[name], seed=SEED)
    prompt = prompt_of(spec.vocab, n)
    cpu = O.Model(spec, n + STEPS + 16, kv_f16=True, threads=threads)
    E, K = spec.cfg.get("experts", 0), spec.cfg.get("experts_used", 0)
    if tape and E:
        # TDecoderRouteTape in record mode: every routed row's picks and
        # weights, in the order the device routes them (layer by layer over
        # each prompt chunk of CHUNK rows, then one row per layer and step)
        cpu.record_routes(spec.cfg["layers"] * (n + STEPS), K)
    for c0 in range(0, n, CHUNK):
        lg = cpu.forward(prompt[c0:c0 + CHUNK])
    top = np.argsort(-lg, kind="stable")[:16]
    first = {"ids": top.tolist(), "logits": [float(lg[i]) for i in top]}
    ids, margins, gaps = [], [], [cpu.route_gap()]
    print(f"[{name}] prompt {n} done in {time.time() - t0:.0f} s", flush=True)
    for i in range(STEPS):
        t = O.argmax(lg)
        ids.append(int(t))
        margins.append(float(lg[t] - np.max(np.delete(lg, t))))
        if i + 1 < STEPS:
            lg = cpu.forward([t])
            gaps.append(cpu.route_gap())
    if tape and E:
        rid, rw = cpu.routes()
        np.savez_compressed(os.path.join(OUT, name + ".routes.npz"),
                            ids=rid.astype(np.uint8 if E <= 256 else np.int32), weights=rw)
    cpu.close()
    rec = {"config": name, "seed": SEED, "prompt_seed": PROMPT_SEED, "prompt_len": n,
           "kv_f16": True, "steps": STEPS, "tokens": ids, "margins": margins,
           "router_gaps": [g if np.isfinite(g) else None for g in gaps],
           "prompt_top16": first}
    os.makedirs(OUT, exist_ok=True)
    with open(os.path.join(OUT, name + ".json"), "w") as f:
        json.dump(rec, f, indent=1)
    print(f"[{name}] {time.time() - t0:.0f} s; tokens {ids[:8]}; min margin "
          f"{min(margins):.3e}", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("configs", nargs="*", default=list(WORKLOADS))
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--tape", action="store_true",
                    help="also write the oracle's expert choice of every routed row (MoE models)")
    a = ap.parse_args()
    for name in a.configs:
        generate(name, a.threads, a.tape)


if __name__ == "__main__":
    main()
