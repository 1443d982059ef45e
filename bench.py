"""Benchmark of mormot.ai.infer.hip on one MI355X.

Workload (BASELINE.json metric "decode tok/s + quant GEMV HBM GB/s (% peak),
Qwen3-30B-A3B-shape Q4_K_M"): configs[3], a Qwen3-30B-A3B-shaped MoE with
Q4_K_M weights (seeded synthetic bytes), a 1024-token prompt, then greedy
decode. A step is one decode token (batch 1); `value` is decode tokens/s.

Beside it, on the same process and device:
- roofline: the decode step's dominant kernel (the MoE layers' gate+up+SwiGLU
  GEMV of the 8 routed experts, Q4_K 768x2048 each, which also routes the
  token), every launch of 32 decode steps timed by its own dispatch's start
  and end events on the library's stream; the decode attention beside it;
- gemv: the configs[1] sweep (Q8_0, Q4_0, Q4_K, Q6_K, MXFP4 over the five
  shapes, batch 1 and 8) in GB/s of algorithmic bytes, each timed group
  cycling > 512 MB of distinct weight copies (beyond the 256 MB MALL);
- stream: a read-only streaming kernel, the achievable HBM read rate;
- cpu_baseline: the CPU oracle (a C restatement of the reference's CPU
  decoder arithmetic) decoding the same model on the host cores.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "mormot2-ai_amd"), os.path.join(ROOT, "tests")]

METRIC = "decode tok/s + quant GEMV HBM GB/s (% peak), Qwen3-30B-A3B-shape Q4_K_M"
HBM_PEAK = 8000.0  # GB/s, MI355X published
INT8_PEAK = 5000.0  # TOP/s, MI355X dense int8 MFMA, published
PROMPTS = {"qwen3-0.6b-q8_0": 32, "qwen3-0.6b-q4_k_m": 512, "qwen3-30b-a3b-q4_k_m": 1024,
           "gpt-oss-20b-mxfp4": 2048}
SWEEP_SHAPES = [(3072, 1024), (1024, 3072), (6144, 2048), (2880, 2880), (151936, 1024)]


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def algo_bytes(dtype, out, cols, rows, mode_q8):
    import infer_hip as H
    w = out * H.row_bytes(dtype, cols)
    x = rows * (cols + cols // 8) if mode_q8 else rows * cols * 4
    return w + x + rows * out * 4


def time_graph(ctx, enqueue, reps):
    """Capture the launches enqueue() makes into a graph, replay it reps
    times between two events; returns ms per replay."""
    import infer_hip as H
    L = H.lib()
    H.check(L.ihip_capture_begin(ctx.h), "capture")
    try:
        enqueue()
    finally:
        H.check(L.ihip_capture_end(ctx.h, 1), "capture end")
    H.check(L.ihip_graph_launch(ctx.h, 1), "graph")
    ctx.sync()
    ctx.record(0)
    for _ in range(reps):
        H.check(L.ihip_graph_launch(ctx.h, 1), "graph")
    ctx.record(1)
    return ctx.elapsed(0, 1) / reps


def stream_peak(ctx):
    import infer_hip as H
    nbytes = 4 << 30
    buf = ctx.alloc(nbytes)
    out = ctx.alloc(256)
    L = H.lib()
    for _ in range(2):
        H.check(L.ihip_enqueue_stream_read(ctx.h, buf.ptr, nbytes, out.ptr))
    ctx.sync()
    ctx.record(0)
    reps = 10
    for _ in range(reps):
        H.check(L.ihip_enqueue_stream_read(ctx.h, buf.ptr, nbytes, out.ptr))
    ctx.record(1)
    ms = ctx.elapsed(0, 1) / reps
    buf.free()
    out.free()
    return nbytes / (ms * 1e-3) / 1e9


def gemv_case(ctx, dtype, out, cols, rows, mode, min_bytes=512 << 20, hot=False):
    """GB/s of one (type, shape, batch, mode): distinct copies of the matrix
    cycled inside a graph, so the weights stream from HBM; hot: the same copy
    every time (a matrix under 256 MB then reads from the MALL/L2)."""
    import infer_hip as H
    L = H.lib()
    wbytes = out * H.row_bytes(dtype, cols)
    ncopies = max(4, -(-min_bytes // wbytes))
    host = H.synth_blocks(dtype, out, cols, out * 7 + cols, -8, -4)
    dev0 = ctx.weight(host, dtype, out, cols)
    stride = (wbytes + 255) // 256 * 256
    big = ctx.alloc(stride * ncopies)
    for i in range(ncopies):
        H.check(L.ihip_copy_async(ctx.h, big.ptr + i * stride, dev0, wbytes))
    x = np.random.default_rng(1).standard_normal((rows, cols)).astype(np.float32)
    dx = ctx.array(x)
    dy = ctx.alloc(rows * out * 4)
    xin, m = dx.ptr, mode
    if mode == H.MODE_Q8:
        kq = 1 if dtype in (H.Q4_K, H.Q6_K) else 0
        dq = ctx.alloc(rows * int(L.ihip_q8_bytes(cols, kq)))
        H.check(L.ihip_enqueue_quantize(ctx.h, dx.ptr, rows, cols, kq, dq.ptr, 0))
        xin, m = dq.ptr, mode | 2
    ctx.sync()

    def enq():
        for i in range(ncopies):
            H.check(L.ihip_enqueue_linear_at(ctx.h, xin, rows, cols, dtype,
                                             big.ptr + (0 if hot else i) * stride, out, dy.ptr, 0, m),
                    "gemv")

    reps = 3
    ms = time_graph(ctx, enq, reps) / ncopies
    nb = algo_bytes(dtype, out, cols, rows, mode == H.MODE_Q8)
    big.free()
    dx.free()
    dy.free()
    if mode == H.MODE_Q8:
        dq.free()
    H.lib().ihip_forget_weights(ctx.h, host.ctypes.data, host.ctypes.data + host.nbytes)
    return nb / (ms * 1e-3) / 1e9, ms * 1e3


def time_direct(ctx, enqueue, reps):
    """The launches of enqueue() made reps times back to back between two
    events, without a graph (the --no-graphs mode a profiled run uses, where
    the host's launch rate bounds the figure); ms per repetition."""
    enqueue()
    ctx.sync()
    ctx.record(0)
    for _ in range(reps):
        enqueue()
    ctx.record(1)
    return ctx.elapsed(0, 1) / reps


def copy_calibration(ctx, nbytes=256 << 20):
    """A plain device copy of known size: the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters of a profile to bytes."""
    import infer_hip as H
    L = H.lib()
    a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
    H.check(L.ihip_copy_async(ctx.h, b.ptr, a.ptr, nbytes), "copy")
    ctx.sync()
    ctx.record(0)
    H.check(L.ihip_copy_async(ctx.h, b.ptr, a.ptr, nbytes), "copy")
    ctx.record(1)
    ms = ctx.elapsed(0, 1)
    a.free()
    b.free()
    return nbytes, 2 * nbytes / (ms * 1e-3) / 1e9


def decode_kernels(ctx, model, spec, first, steps, past):
    """The decode step's own kernels, timed live: `steps` decode steps with
    direct launches (the graph's kernels, launched one by one), every launch
    of the dominant kernel - the MoE layers' gate+up+SwiGLU expert GEMV that
    also routes the token (or, for a dense model, the FFN gate+up+SwiGLU
    GEMV) - timed by its own dispatch's start and end events on the
    library's stream; then the same for the decode attention. Returns the
    per-launch averages and the algorithmic bytes per launch."""
    import infer_hip as H
    c = spec.cfg
    # experts alone (MoE) or beside a dense FFN (Gemma 4): the experts'
    # self-routed gate/up launch
    moe = c.get("moe", False) or c.get("experts", 0) > 0
    act = "GeGLU" if c.get("family") == "gemma4" else "SwiGLU"
    Hd, hd = c["hidden"], c["head_dim"]
    L0 = spec.layers[0]
    if moe:
        E, K, FI = c["experts"], c["experts_used"], c["expert_ffn"]
        gt = L0.exp_gate.dtype
        # both matrices of K experts, the normed row as the router's launch
        # quantized it (Q8_K or Q8_0 codes and a float scale per 32 values),
        # the router logits, the K x FI outputs, the picks and their weights
        wb = 2 * K * FI * H.row_bytes(gt, Hd)
        xrow = 2 * Hd * 4 if c.get("family") == "gemma4" else Hd + 4 * (Hd // 32)
        nb = wb + xrow + E * 4 + K * FI * 4 + K * 8
        if L0.exp_gate_bias.data:
            nb += 2 * K * FI * 4
        what = f"gate+up+{act} of {K} routed experts ({FI}x{Hd}, {H.NAMES[gt]}), route in-launch"
    else:
        FI, gt = c["ffn"], L0.gate.dtype
        wb = 2 * FI * H.row_bytes(gt, Hd)
        nb = wb + 2 * Hd * 4 + FI * 4
        what = f"FFN gate+up+{act} ({FI}x{Hd}, {H.NAMES[gt]})"
    # (the MoE experts read the router launch's quantized row: no norm of their own)
    dom_name = f"gemv_{H.NAMES[gt].lower()}_q8_{'' if moe and c.get('family') != 'gemma4' else 'norm_'}glu"
    kvw = c["kv_heads"] * hd
    out = {}
    model.use_graphs(False)
    tok = first
    for key, prefix in (("dominant", dom_name), ("attention", "attention_")):
        ctx.kernel_timer(prefix, capacity=steps * c["layers"] + 64)
        ids = model.decode(tok, steps)
        n, ms = ctx.kernel_timer_read()
        ctx.kernel_timer(None)
        # the cache length averaged over the timed steps (keys read per launch)
        keys = past + 1 + (steps - 1) / 2.0
        past += steps
        tok = int(ids[-1])
        out[key] = {"prefix": prefix, "launches": n, "avg_us": ms * 1e3 / max(n, 1)}
        if key == "attention":
            # the window layers read fewer keys; configs without windows read all
            out[key]["keys_avg"] = keys
    # every kernel of `steps` steps: the per-token breakdown
    # (the unfused layers of Qwen3.5 and Gemma 4 launch up to ~24 kernels each)
    ctx.kernel_timer("*", capacity=min(60000, steps * (24 * c["layers"] + 32)))
    ids = model.decode(tok, steps)
    rep = ctx.kernel_timer_report()
    ctx.kernel_timer(None)
    past += steps
    tok = int(ids[-1])
    out["per_token"] = {k: {"launches": round(n / steps, 2), "avg_us": round(ms * 1e3 / n, 2),
                            "us_per_token": round(ms * 1e3 / steps, 1)}
                        for k, (n, ms) in sorted(rep.items(), key=lambda kv: -kv[1][1])}
    model.use_graphs(True)
    d = out["dominant"]
    # (a model whose FFN runs otherwise launches no such kernel: 0, and the
    # per-token breakdown says what ran)
    d.update({"kernel": dom_name, "what": what, "bytes_per_launch": nb, "weight_bytes": wb,
              "GBps": nb / (d["avg_us"] * 1e-6) / 1e9 if d["launches"] else 0.0})
    a = out["attention"]
    qw = c["heads"] * hd
    abytes = int(a["keys_avg"] * kvw * 2 * 2 + qw * 4 * 2 + kvw * 4 * 2)
    if not c.get("window") and not c.get("family") and a["launches"]:
        a.update({"bytes_per_launch": abytes, "GBps": abytes / (a["avg_us"] * 1e-6) / 1e9})
    return out, tok, past


PROFILED = {  # roofline kernel -> its committed counter profile
    "gemv_q4_k_q8_glu": "gemv_q4_k_q8_glu_route_8x768x2048_traffic.txt",
}


def profiled_traffic(kernel):
    """HBM bytes per launch of the roofline kernel from the committed counter
    profile (FETCH_SIZE + WRITE_SIZE, each scaled by a copy of known size),
    or None when there is none for this kernel."""
    if kernel not in PROFILED:
        return None
    path = os.path.join(ROOT, "profiles", PROFILED[kernel])
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except (OSError, ValueError):
        pass
    return None


def cpu_baseline(spec, prompt, steps, thread_counts, runs=3):
    """The CPU decoder on TInferCpuFastBackend's default mode (oracle/fast.c:
    AVX2 Linear on work items of 16 outputs over a thread pool, exact
    K-quant super-block sums, the float lanes of Q8DotF32x4x2, the fast
    attention) on the host cores: the whole prompt, one warm-up token, then,
    per thread count, the best of `runs` timed runs of `steps` tokens (as
    linear-bench times the best of 3 after a warm-up). Returns the prefill
    seconds and {threads: tok/s}."""
    import oracle_lib as O
    if not O.fast_available():
        return None, {}
    m = O.Model(spec, len(prompt) + 2 + len(thread_counts) * runs * steps + 2, kv_f16=True,
                threads=thread_counts[0], fast=True)
    t0 = time.perf_counter()
    tok = O.argmax(m.forward(prompt))
    prefill_s = time.perf_counter() - t0
    tok = O.argmax(m.forward([tok]))
    rates = {}
    for th in thread_counts:
        m.set_threads(th)
        best = 0.0
        for _ in range(runs):
            t0 = time.perf_counter()
            for _ in range(steps):
                tok = O.argmax(m.forward([tok]))
            best = max(best, steps / (time.perf_counter() - t0))
        rates[th] = best
    m.close()
    return prefill_s, rates


def cpu_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=None,
                    help="prompt tokens (default: the config's BASELINE workload)")
    ap.add_argument("--config", default="qwen3-30b-a3b-q4_k_m")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--sample-steps", type=int, default=32,
                    help="decode steps with device sampling after the greedy ones (0: none)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-f32", action="store_true", help="skip the F32-mode decode leg")
    ap.add_argument("--kv-f32", action="store_true")
    ap.add_argument("--no-graphs", action="store_true",
                    help="direct launches per decode step (the profiler cannot trace graphs)")
    args = ap.parse_args()
    if args.prompt is None:
        # the BASELINE workloads: configs[0] 32, configs[2] 512, configs[3]
        # 1024, configs[4] 2048 prompt tokens
        args.prompt = PROMPTS.get(args.config, 1024)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"{args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import infer_hip as H
    from infer_hip import models

    ctx = H.Context(0)
    dev_name, dev_mem, cus = ctx.info()
    log("device", dev_name, dev_mem >> 30, "GiB", cus, "CUs")
    stream = stream_peak(ctx)
    log(f"stream read {stream:.0f} GB/s")
    copy_bytes, copy_gbps = copy_calibration(ctx)
    log(f"copy {copy_bytes} B (the counter calibration): {copy_gbps:.0f} GB/s read+write")

    t = time.time()
    spec = models.Spec(models.CONFIGS[args.config], seed=1)
    log(f"synthetic {args.config} built in {time.time() - t:.1f}s")
    max_tokens = args.prompt + args.warmup + args.steps + args.sample_steps + 4 + 96 + 16
    t = time.time()
    model = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=not args.kv_f32, max_tokens=max_tokens)
    log(f"uploaded in {time.time() - t:.1f}s")
    if args.no_graphs:
        model.use_graphs(False)
    prompt = np.random.default_rng(2024).integers(0, spec.vocab, args.prompt).astype(np.int32)
    ctx.sync()
    # the first prefill pays each kernel's first use (code object setup): it
    # is reported apart; prefill_tok_s times the same prompt again after a reset
    t = time.perf_counter()
    lg = model.forward(prompt)
    cold_s = time.perf_counter() - t
    model.reset()
    ctx.sync()
    t = time.perf_counter()
    lg = model.forward(prompt)
    prefill_s = time.perf_counter() - t
    first = int(np.argmax(lg))
    log(f"prefill {args.prompt} tokens {prefill_s * 1e3:.1f} ms (first prefill {cold_s * 1e3:.1f} ms)")
    ids = model.decode(first, args.warmup)
    ctx.sync()
    t0 = time.perf_counter()
    ids2 = model.decode(int(ids[-1]), args.steps)
    ctx.sync()
    dt = time.perf_counter() - t0
    tok_s = args.steps / dt
    log(f"decode {args.steps} steps: {dt * 1e3 / args.steps:.3f} ms/token, {tok_s:.1f} tok/s")
    # the same decode with draws of a TInferSampler (temperature 0.8, top-k 40,
    # top-p 0.95) made on the device inside the graph: the sampler's cost
    sampled = None
    if args.sample_steps > 0:
        model.sampling(temperature=0.8, top_k=40, top_p=0.95, seed=1)
        ids3 = model.decode(int(ids2[-1]), 4)
        ctx.sync()
        t0 = time.perf_counter()
        model.decode(int(ids3[-1]), args.sample_steps)
        ctx.sync()
        st = (time.perf_counter() - t0) / args.sample_steps
        sampled = {"tok_s": round(1.0 / st, 1), "ms_per_token": round(st * 1e3, 4),
                   "settings": "temperature 0.8, top_k 40, top_p 0.95", "steps": args.sample_steps}
        log(f"sampled decode {args.sample_steps} steps: {st * 1e3:.3f} ms/token, {1.0 / st:.1f} tok/s")
        model.sampling()
    wbytes = spec.weight_bytes_per_token()
    # the decode step's dominant kernel and its attention, timed live
    past = args.prompt + args.warmup + args.steps + (4 + args.sample_steps if sampled else 0)
    kt, _, _ = decode_kernels(ctx, model, spec, int(ids2[-1]), 32, past)
    dom = kt["dominant"]
    log("dominant kernel", dom)
    log("attention", kt["attention"])
    for k, v in kt["per_token"].items():
        log(f"  {k:40s} {v}")
    model.close()

    # the same decode in the reference GPU's own contract (IHIP_MODE_F32: float
    # activations, each code dequantized exactly, f32 sums per group;
    # linear.cu:1-6), after the same prompt
    f32_mode = None
    if not args.no_f32:
        mf = H.Model(ctx, spec, mode=H.MODE_F32, kv_f16=not args.kv_f32, max_tokens=max_tokens)
        t = time.perf_counter()
        lgf = mf.forward(prompt)
        f32_prefill = time.perf_counter() - t
        idf = mf.decode(int(np.argmax(lgf)), 8)
        ctx.sync()
        t = time.perf_counter()
        mf.decode(int(idf[-1]), 64)
        ctx.sync()
        ft = (time.perf_counter() - t) / 64
        mf.close()
        f32_mode = {"tok_s": round(1.0 / ft, 1), "ms_per_token": round(ft * 1e3, 4), "steps": 64,
                    "prefill_ms": round(f32_prefill * 1e3, 1),
                    "arithmetic": "f32 activations x exactly dequantized codes, f32 group sums"}
        log(f"f32-mode decode 64 steps: {ft * 1e3:.3f} ms/token, {1.0 / ft:.1f} tok/s "
            f"(prefill {f32_prefill * 1e3:.0f} ms)")

    sweep, mall_hot = {}, {}
    if not args.no_sweep:
        for dtype in (H.Q8_0, H.Q4_0, H.Q4_K, H.Q6_K, H.MXFP4):
            for out, cols in SWEEP_SHAPES:
                if cols % H.BLOCK[dtype][0]:
                    continue  # 2880 is no whole number of 256-value super-blocks
                for rows, mode in ((1, H.MODE_Q8), (1, H.MODE_F32), (8, H.MODE_Q8),
                                   (512, H.MODE_Q8)):
                    gbps, us = gemv_case(ctx, dtype, out, cols, rows, mode)
                    key = f"{H.NAMES[dtype]} {out}x{cols} b{rows} {'q8' if mode else 'f32'}"
                    if rows >= 16:
                        # the MFMA GEMM: int8 operations per second against the
                        # dense int8 MFMA peak (the instruction it runs on)
                        tops = 2.0 * rows * cols * out / (us * 1e-6) / 1e12
                        sweep[key] = {"TOPs": round(tops, 1), "us": round(us, 2),
                                      "mfma_frac": round(tops / INT8_PEAK, 4)}
                    else:
                        sweep[key] = {"GBps": round(gbps, 1), "us": round(us, 2),
                                      "frac": round(gbps / HBM_PEAK, 3)}
                    log(key, sweep[key])
                    if rows == 1 and mode == H.MODE_Q8:
                        # the same launch with the matrix cache-resident
                        # (labelled apart: not an HBM figure)
                        hg, hus = gemv_case(ctx, dtype, out, cols, rows, mode, hot=True)
                        mall_hot[key] = {"GBps": round(hg, 1), "us": round(hus, 2)}

    cpu = None
    if not args.no_cpu:
        # every core this process may run on (its affinity mask: the box's
        # CPU share), and the reference's default pool size of it
        # ((cores * 2 + 2) / 3, backend.cpu.pas:1989)
        cores = max(1, len(os.sched_getaffinity(0)))
        nproc = os.cpu_count() or cores
        ref_threads = max(1, (cores * 2 + 2) // 3)
        t = time.time()
        cpu_prefill_s, rates = cpu_baseline(spec, prompt, 8, [cores, ref_threads])
        if rates:
            cpu = {"value": round(rates[cores], 3), "unit": "tok/s", "cores": cores, "kind": "port",
                   "affinity_cores": cores, "host_cpus": nproc,
                   "variant": "avx2",
                   "value_ref_threads": round(rates[ref_threads], 3), "ref_threads": ref_threads,
                   "prefill_tok_s": round(len(prompt) / cpu_prefill_s, 1),
                   "sample": f"{args.config} decode after the same {len(prompt)}-token prompt: "
                             f"best of 3 runs of 8 tokens after a warm-up token, at {cores} and "
                             f"at {ref_threads} threads; TInferCpuFastBackend's default mode "
                             f"restated in C with AVX2/FMA (oracle/fast.c: tiles of 16 outputs "
                             f"over an OpenMP pool, exact K-quant sums, Q8DotF32x4x2 float "
                             f"lanes, the fast attention) on {cpu_name()}; {cores} threads = "
                             f"every core of this process's affinity mask ({nproc} CPUs on "
                             f"the host)"}
            log(f"cpu baseline {rates[cores]:.3f} tok/s ({cores} threads), "
                f"{rates[ref_threads]:.3f} ({ref_threads} threads), prefill "
                f"{cpu_prefill_s:.1f} s, in {time.time() - t:.1f}s")

    big = [v["GBps"] for k, v in sweep.items() if "151936" in k and "b1 q8" in k]
    result = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 (Q8_K activations x Q4_K/Q6_K codes, int32 sums, f64 scaling)",
        "data": "synthetic (seeded random Q4_K_M bytes of the architecture)",
        "config": {"workload": f"{args.config} greedy decode after a {args.prompt}-token prompt",
                   "prompt": args.prompt, "kv_cache": "f32" if args.kv_f32 else "f16",
                   "weight_bytes_per_token": wbytes, "parallelism": "single GPU",
                   "graphs": not args.no_graphs},
        "prefill_tok_s": round(args.prompt / prefill_s, 1),
        "prefill_first_ms": round(cold_s * 1e3, 2),
        "sampled_decode": sampled,
        "f32_mode_decode": f32_mode,
        "decode_weight_GBps": round(wbytes * tok_s / 1e9, 1),
        "roofline": {"bound": "hbm", "achieved": round(dom["GBps"], 1), "peak": HBM_PEAK,
                     "unit": "GB/s", "frac": round(dom["GBps"] / HBM_PEAK, 4),
                     "traffic": profiled_traffic(dom["kernel"]),
                     "kernel": dom["kernel"] + "*", "what": dom["what"],
                     "bytes_per_launch": dom["bytes_per_launch"], "avg_us": round(dom["avg_us"], 3),
                     "launches_timed": dom["launches"]},
        "attention": {k: (round(v, 3) if isinstance(v, float) else v)
                      for k, v in kt["attention"].items()},
        "decode_kernels": kt["per_token"],
        "stream_read_GBps": round(stream, 1),
        "copy_GBps": round(copy_gbps, 1),
        "gemv_head_151936x1024_b1_GBps": big,
        "gemv": sweep,
        # batch-1 GEMVs replaying one copy of the matrix: cache-resident
        # (MALL/L2) for matrices under 256 MB, not HBM bandwidth
        "gemv_mall_hot": mall_hot,
        "cpu_baseline": cpu,
        "device": dev_name,
    }
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
    # every device buffer is freed and the line is printed: leave without
    # waiting on interpreter teardown (the CPU baseline's OpenMP pool and the
    # HIP runtime's threads), so no process of the run outlives it - except
    # under rocprofv3, whose results are written by the exit handlers
    sys.stderr.flush()
    profiled = any(k.startswith("ROCP") for k in os.environ) or \
        "rocprof" in os.environ.get("LD_PRELOAD", "")
    if not profiled:
        os._exit(0)
