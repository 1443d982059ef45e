"""Phase stamps of the decode kernels, from the timing build
(IHIP_TRACE=1 python mormot2-ai_amd/build.py -> libmormot_ai_hip_trace.so).

Thread 0 of every block of an instrumented kernel records the 100 MHz clock
at numbered phases (IHIP_STAMP in the kernels). This decodes a synthetic
model of a BASELINE configuration after a prompt, with direct launches (no
graph), traces every launch of each kernel name prefix over a few decode
steps, and prints per phase the median / 10th / 90th percentile over blocks
and launches of the time since the launch's earliest block started (us).

  python mormot2-ai_amd/phase_stamps.py [config] [prefix,prefix,...] [prompt] [group]

With a group size, the medians and 90th percentiles of phases 0, 1, 2, 4 and
5 are also printed for every group of that many consecutive blocks (in
dispatch order: the matrices of a several-matrix launch, an expert slot's
blocks, the key ranges of the decode attention).

Phases of the one-row GEMV (linear.hip gemv, R = 1): 0 block start, 6 the
activation row's loads issued (self-routed experts: after the router logits),
7 the block's expert picked (self-routed only), 1 the first weight loads
issued, 2 the row staged in LDS, 3 the row's groups in registers, 4 after
each wave step's sums, 5 the block's last store. Of the expert down+combine
(linear.hip gemv_cmb): 0 start, 6 the slot rows' loads issued, 1 the first
weight loads issued (after the expert ids), 2 the rows staged in LDS, 4 after
each tile's combine, 5 the block's end. Of the decode attention
(ops.hip attention_one): 0 start, 1 every load issued, 2 head norms, RoPE and
the cache store done, 3 the softmax done, 4 the weighted values in LDS, 5 the
merge started (the head's last range block), 6 the merge done.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
os.environ.setdefault("IHIP_LIB", os.path.join(HERE, "libmormot_ai_hip_trace.so"))

import infer_hip as H  # noqa: E402
from infer_hip import models  # noqa: E402

MAXB = 1 << 14  # blocks per traced launch


def main():
    cfg = sys.argv[1] if len(sys.argv) > 1 else "qwen3-30b-a3b-q4_k_m"
    prefixes = (sys.argv[2].split(",") if len(sys.argv) > 2 else
                ["gemv_q4_k_q8_norm_glu", "attention_one", "gemv_q4_k_q6_k_q8_norm",
                 "gemv_q4_k_q8_u4", "gemv_f32_q8_norm_rows"])
    plen = int(sys.argv[3]) if len(sys.argv) > 3 else 1024
    group = int(sys.argv[4]) if len(sys.argv) > 4 else 0
    ctx = H.Context(0)
    spec = models.Spec(models.CONFIGS[cfg], seed=1)
    m = H.Model(ctx, spec, mode=H.MODE_Q8, kv_f16=True, max_tokens=plen + 64)
    m.use_graphs(False)
    prompt = np.random.default_rng(1).integers(0, spec.vocab, plen).astype(np.int32)
    tok = int(np.argmax(m.forward(prompt)))
    tok = int(m.decode(tok, 4)[-1])
    L = H.lib()
    stride = MAXB * 64
    count = spec.cfg["layers"] * 3
    buf = ctx.alloc(stride * count)
    print(f"{cfg}: prompt {plen}, 3 decode steps per kernel, us since the launch's first block",
          flush=True)
    for p in prefixes:
        buf.upload(np.zeros(stride * count // 8, np.uint64))
        H.check(L.ihip_trace_buffer(ctx.h, buf.ptr, stride, count, p.encode()), "trace")
        tok = int(m.decode(tok, 3)[-1])
        H.check(L.ihip_trace_buffer(ctx.h, 0, 0, 0, None), "trace off")
        ctx.sync()
        a = buf.download(np.uint64, stride * count // 8).reshape(count, MAXB, 8).astype(np.int64)
        rows = []
        for k in range(count):
            s = a[k]
            used = s[:, 0] > 0
            if not used.any():
                break
            s = s[used]
            rows.append(np.where(s > 0, (s - s[:, 0].min()) * 0.01, np.nan))
        print(f"== {p}*: {len(rows)} launches, {rows[0].shape[0] if rows else 0} blocks each",
              flush=True)
        if not rows:
            continue
        allr = np.concatenate(rows)
        for i in (0, 6, 7, 1, 2, 3, 4, 5):
            col = allr[:, i]
            col = col[~np.isnan(col)]
            if col.size:
                print(f"  phase {i}: median {np.median(col):6.2f}  p10 {np.percentile(col, 10):6.2f}"
                      f"  p90 {np.percentile(col, 90):6.2f}  max {col.max():6.2f}  blocks {col.size}")
        print(f"  last stamp of a launch: median {np.median([np.nanmax(r) for r in rows]):.2f} us",
              flush=True)
        if group > 0:
            R = np.stack(rows)  # launches x blocks x 8
            for g0 in range(0, R.shape[1], group):
                part = R[:, g0:g0 + group, :]
                cols = []
                for i in (0, 1, 2, 4, 5):
                    v = part[:, :, i]
                    v = v[~np.isnan(v)]
                    cols.append(f"p{i} {np.median(v):5.2f}/{np.percentile(v, 90):5.2f}" if v.size
                                else f"p{i}   -  /  -  ")
                print(f"  blocks {g0:4d}-{min(R.shape[1], g0 + group) - 1:4d}: " + "  ".join(cols),
                      flush=True)
    m.close()
    ctx.close()
    sys.stdout.flush()
    os._exit(0)


if __name__ == "__main__":
    main()
