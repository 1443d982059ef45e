"""Parity over the exact grid the benchmark's GEMV/GEMM sweep times
(the reference's harness is demos/infer/linear-bench.lpr:
181-198): the five formats Q8_0, Q4_0, Q4_K, Q6_K and MXFP4 on the matrices
3072x1024, 1024x3072, 6144x2048, 2880x2880 and 151936x1024 (rows x cols), with
the sweep's own seeded weights (uniform codes, block scales in [2^-8, 2^-4]:
infer_hip.synth_blocks with the bench's seeds) and float activations ~N(0,1),
at batch 1, 8 and 512, through the C-ABI Linear:

- Q8 mode (the reference CPU's arithmetic) against the oracle's Linear: at
  most 1 ulp apart (only the order of a double sum differs) and at most one
  value in a thousand differing; batch 1 runs on the one-row GEMV, batch 8 on
  gemm8 or the 8-row GEMVs, batch 512 on the MFMA GEMM;
- F32 mode at batch 1 (the reference GPU's arithmetic) against the oracle's
  F32 Linear: relative L2 and max-norm error <= 1e-5.

For the 151936-output head at batch 512 the oracle computes a seeded subset
of 4096 output rows (the device computes all of them); every other case is
compared whole."""
import os

import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O
from golden_io import rel_error, rel_l2

pytestmark = pytest.mark.gpu

FMTS = [H.Q8_0, H.Q4_0, H.Q4_K, H.Q6_K, H.MXFP4]
SHAPES = [(3072, 1024), (1024, 3072), (6144, 2048), (2880, 2880), (151936, 1024)]
THREADS = max(1, len(os.sched_getaffinity(0)))
SUBSET = 4096


def ulp_diff(a, b):
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    yield c
    c.close()


# 2880 columns are no whole number of the K-quants' 256-value super-blocks:
# the sweep (and the formats) have no Q4_K / Q6_K matrix of that width
GRID = [(d, o, c) for d in FMTS for o, c in SHAPES if c % H.BLOCK[d][0] == 0]


@pytest.mark.timeout(600)
@pytest.mark.parametrize("dtype,out,cols", GRID)
def test_sweep_grid(ctx, dtype, out, cols):
    # the bench's own matrix of this format and shape (bench.py sweep seeds)
    w = H.synth_blocks(dtype, out, cols, out * 7 + cols, -8, -4)
    rb = H.row_bytes(dtype, cols)
    rng = np.random.default_rng(out + cols + dtype)
    name = f"{H.NAMES[dtype]} {out}x{cols}"
    for rows in (1, 8, 512):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        print(f"[{name}] batch {rows}", flush=True)
        y = ctx.linear(x, w, dtype, out, None, mode=H.MODE_Q8)
        if rows == 512 and out > 16384:
            idx = np.sort(np.random.default_rng(7).choice(out, SUBSET, replace=False))
            wsub = np.ascontiguousarray(w.reshape(out, rb)[idx]).reshape(-1)
            ref = O.linear(x, wsub, dtype, SUBSET, threads=THREADS)
            y = np.ascontiguousarray(y[:, idx])
        else:
            ref = O.linear(x, w, dtype, out, threads=THREADS)
        u = ulp_diff(y, ref)
        assert u.max() <= 1, (name, rows, int(u.max()))
        assert np.count_nonzero(u) <= max(2, u.size // 1000), (name, rows, int(np.count_nonzero(u)))
        if rows == 1:
            yf = ctx.linear(x, w, dtype, out, None, mode=H.MODE_F32)
            rf = O.linear(x, w, dtype, out, threads=THREADS, f32=True)
            assert rel_l2(yf, rf) <= 1e-5 and rel_error(yf, rf) <= 1e-5, (name, rel_l2(yf, rf))
    # the weight cache is keyed by host address: forget this matrix before
    # its array is freed
    H.lib().ihip_forget_weights(ctx.h, H._p(w), H.C.c_void_p(w.ctypes.data + w.nbytes))
