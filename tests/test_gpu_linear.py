"""GPU parity of the dequant and the Linear kernels through the C-ABI
(LinearMatchesReference and LinearIdsMatchesReference of the reference,
tests/test.infer.cuda.pas:714-967, 2333-2447):

- tier 1: the device dequant of every type equals the oracle's InferRowToF32
  bit for bit;
- tier 2 (IHIP_MODE_F32): RelError (max|a-b|/max|b|) <= 1e-5 and relative L2
  <= 1e-5 against the double Linear over InferRowToF32 weights;
- Q8 mode: the CPU reference Linear's bits (x quantized to Q8_0 / Q8_K, exact
  integer sums, double scaling), allowing a 1-ulp difference only where the
  order of a double sum differs - counted and bounded.
"""
import os

import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O
from golden_io import GoldenSet, compare, rel_error, rel_l2

pytestmark = pytest.mark.gpu

BLOCK_FMTS = [H.Q8_0, H.Q4_0, H.MXFP4, H.Q5_0, H.Q5_1, H.Q4_K, H.Q6_K]
ALL_FMTS = BLOCK_FMTS + [H.F32, H.BF16, H.F16]
# (rows, in, out): the LinearMatchesReference shapes that fit the block sizes
SHAPES = [(1, 256, 70001), (70, 512, 130), (1, 896, 65), (1, 2560, 37), (3, 1024, 515),
          (8, 768, 300), (1, 3072, 1024), (9, 2048, 257), (1, 2880, 129)]


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    print("device:", c.info(), flush=True)
    yield c
    c.close()


def weights(dtype, out, cols, seed):
    if dtype in (H.F32, H.BF16, H.F16):
        return H.synth_normal(dtype, out, cols, seed, 0.5)
    return H.synth_blocks(dtype, out, cols, seed, -8, -4)


def fits(dtype, cols):
    return cols % H.BLOCK[dtype][0] == 0 and cols % 32 == 0


@pytest.mark.parametrize("dtype", ALL_FMTS)
def test_dequant_bit_exact(ctx, dtype):
    for out, cols in ((37, 512), (5, 2816), (129, 3072)):
        if not fits(dtype, cols):
            continue
        w = weights(dtype, out, cols, out + cols)
        dw = ctx.weight(w, dtype, out, cols)
        y = ctx.alloc(out * cols * 4)
        H.check(H.lib().ihip_enqueue_dequant(ctx.h, dw, dtype, out, cols, 0, out, y.ptr))
        got = y.download(np.float32, out * cols).reshape(out, cols)
        ref = O.dequant(w, dtype, out, cols)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (H.NAMES[dtype], out, cols)
        y.free()


@pytest.mark.parametrize("dtype", [H.MXFP4])
def test_mxfp4_edge_exponents(ctx, dtype):
    # test.infer.cuda.pas:840-864: exponents {0, 1, 2, 127, 128, 200}, x = 1
    out, cols = 6, 64
    w = H.synth_blocks(H.MXFP4, out, cols, 3).reshape(out, 2, 17)
    for i, e in enumerate((0, 1, 2, 127, 128, 200)):
        w[i, :, 0] = e
    w = w.ravel().copy()
    x = np.ones((1, cols), np.float32)
    y = ctx.linear(x, w, H.MXFP4, out)
    ref = O.linear(x, w, H.MXFP4, out, f32=True)
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("mode", [H.MODE_F32, H.MODE_Q8])
def test_zero_codes_at_extreme_scales(ctx, mode):
    # blocks whose values are all zero (-0 included) under the largest scales
    # - MXFP4 exponents 255, 254, 200, 0, 1 (the tiny gpt-oss checkpoint holds
    # a -0 block with exponent 255), Q8_0 / Q4_0 / Q5_0 at fp16 scale 65504 -
    # give exact zero rows, with random activations; the other rows as the CPU
    rng = np.random.default_rng(11)
    cols = 64
    x = rng.standard_normal((3, cols)).astype(np.float32)
    cases = []
    w = H.synth_blocks(H.MXFP4, 6, cols, 5).reshape(6, 2, 17)
    for i, e in enumerate((255, 254, 200, 0, 1)):
        w[i, :, 0] = e
        w[i, :, 1:] = 0x88 if i % 2 == 0 else 0x00  # -0 or +0 codes
    cases.append((H.MXFP4, w.ravel().copy(), 6))
    for dt, zero in ((H.Q8_0, 0x00), (H.Q4_0, 0x88)):
        bs = H.BLOCK[dt][1]
        w = H.synth_blocks(dt, 4, cols, 6).reshape(4, 2, bs)
        w[:2, :, 0:2] = np.frombuffer(np.float16(65504).tobytes(), np.uint8)
        w[:2, :, 2:] = zero
        cases.append((dt, w.ravel().copy(), 4))
    w = H.synth_blocks(H.Q5_0, 4, cols, 7).reshape(4, 2, 22)
    w[:2, :, 0:2] = np.frombuffer(np.float16(65504).tobytes(), np.uint8)
    w[:2, :, 2:6] = 0xFF   # the fifth bits set and nibbles 0: q = 16, value 0
    w[:2, :, 6:] = 0x00
    cases.append((H.Q5_0, w.ravel().copy(), 4))
    for dt, w, out in cases:
        y = ctx.linear(x, w, dt, out, mode=mode)
        ref = O.linear(x, w, dt, out, f32=(mode == H.MODE_F32))
        zero_rows = 5 if dt == H.MXFP4 else 2
        assert np.all(y[:, :zero_rows] == 0), (H.NAMES[dt], y[:, :zero_rows])
        assert np.all(ref[:, :zero_rows] == 0)
        assert rel_error(y, ref) <= 1e-5, (H.NAMES[dt], mode)


@pytest.mark.parametrize("dtype", ALL_FMTS)
def test_linear_f32_mode(ctx, dtype):
    rng = np.random.default_rng(7)
    for rows, cols, out in SHAPES:
        if not fits(dtype, cols):
            continue
        w = weights(dtype, out, cols, rows * 31 + cols + out)
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        b = rng.standard_normal(out).astype(np.float32)
        y = ctx.linear(x, w, dtype, out, b, mode=H.MODE_F32)
        ref = O.linear(x, w, dtype, out, b, f32=True)
        e1, e2 = rel_error(y, ref), rel_l2(y, ref)
        assert e1 <= 1e-5 and e2 <= 1e-5, (H.NAMES[dtype], rows, cols, out, e1, e2)
        # the second, cached call gives the same bits (test.infer.cuda.pas:833-837)
        y2 = ctx.linear(x, w, dtype, out, b, mode=H.MODE_F32)
        assert np.array_equal(y, y2)


def ulp_diff(a, b):
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("dtype", ALL_FMTS)
def test_linear_q8_mode_cpu_bits(ctx, dtype):
    rng = np.random.default_rng(9)
    total, differ = 0, 0
    for rows, cols, out in SHAPES:
        if not fits(dtype, cols):
            continue
        w = weights(dtype, out, cols, rows * 17 + cols + out)
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        b = rng.standard_normal(out).astype(np.float32)
        y = ctx.linear(x, w, dtype, out, b, mode=H.MODE_Q8)
        ref = O.linear(x, w, dtype, out, b)
        u = ulp_diff(y, ref)
        assert u.max() <= 1, (H.NAMES[dtype], rows, cols, out, int(u.max()))
        total += u.size
        differ += int(np.count_nonzero(u))
    assert differ <= max(2, total // 1000), (differ, total)


# batches of 2..15 rows on the batch GEMV (rows staged in LDS, the 8 rows'
# sums reduced transposed across the lanes of an output): every row has the
# bits of that row run alone, ragged last chunks included, at input widths
# whose lanes per output run from 2 to 64
@pytest.mark.parametrize("dtype", BLOCK_FMTS)
def test_batch_rows_bits_of_one_row(ctx, dtype):
    rng = np.random.default_rng(21)
    for cols in (64, 256, 1024, 3072):
        if not fits(dtype, cols):
            continue
        for rows, out in ((2, 300), (3, 1024), (5, 97), (8, 640), (11, 300), (15, 130)):
            w = weights(dtype, out, cols, rows * 7 + cols + out)
            x = rng.standard_normal((rows, cols)).astype(np.float32)
            b = rng.standard_normal(out).astype(np.float32) if rows % 2 else None
            y = ctx.linear(x, w, dtype, out, b, mode=H.MODE_Q8)
            for r in range(rows):
                one = ctx.linear(x[r:r + 1], w, dtype, out, b, mode=H.MODE_Q8)
                assert np.array_equal(y[r].view(np.uint32), one[0].view(np.uint32)), \
                    (H.NAMES[dtype], rows, cols, out, r)


# small batches whose 128-output tiles fill the chip run on the int8 matrix
# cores (gemm8: 8 rows per block, the weights read once per 8 rows); the
# last row chunk partial, rows past it absent
GEMM8_SHAPES = [(8, 256, 40000), (3, 512, 33000), (13, 1024, 32896), (2, 2048, 36000)]


@pytest.mark.parametrize("dtype", BLOCK_FMTS)
def test_gemm8_q8_mode_cpu_bits(ctx, dtype):
    rng = np.random.default_rng(11)
    total, differ = 0, 0
    for rows, cols, out in GEMM8_SHAPES:
        if not fits(dtype, cols):
            continue
        w = weights(dtype, out, cols, rows * 31 + cols + out)
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        b = rng.standard_normal(out).astype(np.float32) if rows != 3 else None
        y = ctx.linear(x, w, dtype, out, b, mode=H.MODE_Q8)
        ref = O.linear(x, w, dtype, out, b)
        u = ulp_diff(y, ref)
        assert u.max() <= 1, (H.NAMES[dtype], rows, cols, out, int(u.max()))
        total += u.size
        differ += int(np.count_nonzero(u))
    assert differ <= max(2, total // 1000), (differ, total)


GEMM_FMTS = [H.Q8_0, H.Q4_0, H.MXFP4, H.Q5_0, H.Q5_1, H.Q4_K, H.Q6_K, H.F32, H.BF16, H.F16]
GEMM_SHAPES = [(16, 256, 64), (64, 2048, 1024), (200, 768, 136), (130, 2560, 100), (40, 2880, 70)]


@pytest.fixture(scope="module")
def gemm_ctx():
    # a context that sends every chunk of 16 rows or more to the GEMM (the
    # default sends chunks of 80 or more; smaller ones go to 8-row GEMVs)
    # (the settings are read when a context is created; the caller's own
    # values come back afterwards)
    saved = {k: os.environ.get(k) for k in ("IHIP_GEMM_MIN_ROWS", "IHIP_GEMM")}
    os.environ["IHIP_GEMM_MIN_ROWS"] = "16"
    os.environ["IHIP_GEMM"] = "1"
    try:
        c = H.Context(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    yield c
    c.close()


@pytest.mark.parametrize("dtype", GEMM_FMTS)
def test_gemm_q8_mode_cpu_bits(gemm_ctx, dtype):
    # chunks of >= 16 rows run on the MFMA GEMM here: exact int32 group sums
    # from the int8 matrix cores, the scales in double, as the CPU; float
    # weights on the f64 matrix cores (exact products, double sums)
    ctx = gemm_ctx
    rng = np.random.default_rng(19)
    total, differ = 0, 0
    for rows, cols, out in GEMM_SHAPES:
        if not fits(dtype, cols):
            continue
        w = weights(dtype, out, cols, rows * 5 + cols + out)
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        b = rng.standard_normal(out).astype(np.float32)
        y = ctx.linear(x, w, dtype, out, b, mode=H.MODE_Q8)
        ref = O.linear(x, w, dtype, out, b)
        u = ulp_diff(y, ref)
        assert u.max() <= 1, (H.NAMES[dtype], rows, cols, out, int(u.max()))
        total += u.size
        differ += int(np.count_nonzero(u))
    assert differ <= max(2, total // 1000), (differ, total)


@pytest.mark.parametrize("name,wkey,ykey,dtype,atol,rtol", [
    ("q8", "linear/weight", "linear/y", H.Q8_0, 1e-5, 1e-5),
    ("q4", "linear/weight", "linear/y", H.Q4_0, 1e-5, 1e-5),
    ("q5", "linear/weight", "linear/y", H.Q5_0, 1e-5, 1e-5),
    ("q51", "linear/weight", "linear/y", H.Q5_1, 2e-3, 2e-4),
    ("mxfp4", "linear/weight", "linear/y", H.MXFP4, 1e-5, 1e-5),
    ("qk", "q4_K/weight", "q4_K/y", H.Q4_K, 1e-4, 1e-5),
    ("qk", "q6_K/weight", "q6_K/y", H.Q6_K, 1e-4, 1e-5)])
def test_linear_q8_mode_golden(ctx, name, wkey, ykey, dtype, atol, rtol):
    # the reference's ggml fixtures, at the reference's tolerances
    g = GoldenSet(name)
    x, b, w, y = g["linear/x"], g["linear/bias"], np.ascontiguousarray(g[wkey]), g[ykey]
    mine = ctx.linear(x, w, dtype, b.size, b, mode=H.MODE_Q8)
    ok, err = compare(mine, y, atol, rtol)
    assert ok, err


@pytest.mark.parametrize("mode", [H.MODE_F32, H.MODE_Q8])
@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_K, H.Q6_K, H.MXFP4, H.BF16])
def test_linear_ids(ctx, dtype, mode):
    # LinearIdsMatchesReference: 5 experts, 4 slots with ids (3, 0, 4, 3), x
    # per slot or shared, with and without a bias
    E, cols, out = 5, 512, 96
    w = weights(dtype, E * out, cols, 77)
    dw = ctx.weight(w, dtype, out, cols, E)
    rng = np.random.default_rng(5)
    ids = np.array([3, 0, 4, 3], np.int32)
    bias = rng.standard_normal((E, out)).astype(np.float32)
    xs = rng.standard_normal((4, cols)).astype(np.float32)
    stride = out * H.row_bytes(dtype, cols)
    dids = ctx.array(ids)
    dx = ctx.array(xs)
    db = ctx.array(bias)
    dy = ctx.alloc(4 * out * 4)
    for per_slot in (1, 0):
        for with_bias in (True, False):
            H.check(H.lib().ihip_enqueue_linear_ids(ctx.h, dx.ptr, cols, dtype, dw, stride, out,
                                                    dids.ptr, 4, per_slot, dy.ptr,
                                                    db.ptr if with_bias else 0, mode))
            got = dy.download(np.float32, 4 * out).reshape(4, out)
            for s in range(4):
                e = ids[s]
                we = w[e * stride:(e + 1) * stride]
                xr = xs[s:s + 1] if per_slot else xs[0:1]
                bb = bias[e] if with_bias else None
                if mode == H.MODE_F32:
                    ref = O.linear(xr, we, dtype, out, bb, f32=True)[0]
                    assert rel_error(got[s], ref) <= 1e-5
                else:
                    ref = O.linear(xr, we, dtype, out, bb)[0]
                    assert ulp_diff(got[s], ref).max() <= 1
    for b in (dids, dx, db, dy):
        b.free()


def test_linear_big_head_shape(ctx):
    # the 151936 x 1024 head at batch 1, both modes
    out, cols = 151936, 1024
    w = H.synth_blocks(H.Q8_0, out, cols, 12)
    x = np.random.default_rng(2).standard_normal((1, cols)).astype(np.float32)
    y = ctx.linear(x, w, H.Q8_0, out, mode=H.MODE_F32)
    ref = O.linear(x, w, H.Q8_0, out, f32=True)
    assert rel_error(y, ref) <= 1e-5
    y = ctx.linear(x, w, H.Q8_0, out, mode=H.MODE_Q8)
    ref = O.linear(x, w, H.Q8_0, out)
    assert ulp_diff(y, ref).max() <= 1


def test_quantize_like_cpu(ctx):
    # the device quantizers give the CPU's codes and scales (Q8_0 ties to
    # even, Q8_K): checked on the ggml fixtures of the reference
    for name, key, kq in (("q8", "quant", 0), ("qk", "q8k", 1)):
        g = GoldenSet(name)
        x = g[f"{key}/x"]
        blocks = g[f"{key}/blocks"]
        rows, cols = x.shape
        dx = ctx.array(x)
        qb = int(H.lib().ihip_q8_bytes(cols, kq))
        dq = ctx.alloc(rows * qb)
        H.check(H.lib().ihip_enqueue_quantize(ctx.h, dx.ptr, rows, cols, kq, dq.ptr, 0))
        got = dq.download(np.uint8, rows * qb).reshape(rows, qb)
        for r in range(rows):
            codes = got[r, :cols].view(np.int8)
            scales = got[r, cols:].view(np.float32)
            if kq == 0:
                ref = blocks[r].reshape(-1, 34)
                assert np.array_equal(codes.reshape(-1, 32), ref[:, 2:].view(np.int8))
                assert np.array_equal(scales, ref[:, :2].copy().view(np.float16).astype(np.float32).ravel())
            else:
                ref = blocks[r].reshape(-1, 292)
                assert np.array_equal(codes.reshape(-1, 256), ref[:, 4:260].view(np.int8))
                d = ref[:, :4].copy().view(np.float32).ravel()
                assert np.array_equal(scales.reshape(-1, 8), np.repeat(d[:, None], 8, axis=1))
        dx.free()
        dq.free()


def test_forget_weights_serves_new(ctx):
    # ForgetWeightsServesNew (test.infer.cuda.pas:3339): host memory rewritten
    # at the same address is served anew once forgotten, stale before
    out, cols = 64, 256
    w = H.synth_blocks(H.Q8_0, out, cols, 1)
    x = np.random.default_rng(3).standard_normal((1, cols)).astype(np.float32)
    y1 = ctx.linear(x, w, H.Q8_0, out)
    w[:] = H.synth_blocks(H.Q8_0, out, cols, 2)
    assert np.array_equal(ctx.linear(x, w, H.Q8_0, out), y1)  # the cached copy
    import ctypes as C
    ep = H.lib().ihip_forget_weights(ctx.h, C.c_void_p(w.ctypes.data),
                                     C.c_void_p(w.ctypes.data + w.nbytes))
    assert ep > 0
    y2 = ctx.linear(x, w, H.Q8_0, out)
    assert rel_error(y2, O.linear(x, w, H.Q8_0, out, f32=True)) <= 1e-5
    assert not np.array_equal(y1, y2)


def test_two_models_at_reused_addresses(ctx):
    # a model forgets its weights when it goes: the next model's host tensors
    # may sit at the same addresses and must not meet the stale copies
    from infer_hip import models
    outs = []
    for seed in (1, 2, 1):
        spec = models.Spec(models.tiny("qwen3-0.6b-q8_0", layers=1, vocab=512, hidden=256,
                                       heads=4, kv_heads=2, head_dim=64, ffn=512), seed=seed)
        m = H.Model(ctx, spec, max_tokens=16)
        outs.append(m.forward([1, 2, 3]))
        ref = O.Model(spec, 16).forward([1, 2, 3])
        m.close()
        del spec
        assert np.abs(outs[-1] - ref).max() <= 1e-5 * np.abs(ref).max()
    assert np.array_equal(outs[0], outs[2]) and not np.array_equal(outs[0], outs[1])


@pytest.fixture(scope="module")
def f8_ctx():
    # MXFP4 chunks of 16 rows or more on the scaled f8f6f4 matrix cores
    saved = {k: os.environ.get(k) for k in ("IHIP_GEMM_MIN_ROWS", "IHIP_GEMM", "IHIP_GEMM_F8")}
    os.environ.update(IHIP_GEMM_MIN_ROWS="16", IHIP_GEMM="1", IHIP_GEMM_F8="1")
    try:
        c = H.Context(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    yield c
    c.close()


def test_gemm_mxfp4_f8f6f4_bits_of_int8(f8_ctx, gemm_ctx):
    # the MXFP4 GEMM on v_mfma_scale_f32_32x32x64_f8f6f4 (e2m1 codes as
    # stored, the activation split q = 16 hi + lo into e4m3 planes) gives the
    # exact group sums the int8 MFMA gives: every output the same bits, and
    # the oracle's to 1 ulp
    rng = np.random.default_rng(31)
    for rows, cols, out in GEMM_SHAPES + [(512, 2880, 2880), (100, 1024, 3000)]:
        w = weights(H.MXFP4, out, cols, rows + cols + out)
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        b = rng.standard_normal(out).astype(np.float32)
        a = f8_ctx.linear(x, w, H.MXFP4, out, b, mode=H.MODE_Q8)
        c = gemm_ctx.linear(x, w, H.MXFP4, out, b, mode=H.MODE_Q8)
        assert np.array_equal(a.view(np.uint32), c.view(np.uint32)), (rows, cols, out)
        if rows <= 200:
            assert ulp_diff(a, O.linear(x, w, H.MXFP4, out, b)).max() <= 1
