"""GPU parity of the layer operations against the CPU oracle (OpsMatchCpu,
RouteMatchesHost of tests/test.infer.cuda.pas:970-1535, 2663-): the device
kernels follow the CPU's arithmetic, so the results must agree to the last
bit up to the order of double sums (max 1 ulp)."""
import numpy as np
import pytest

import infer_hip as H
import oracle_lib as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = H.Context(0)
    yield c
    c.close()


def ulp(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return int(np.abs(ia - ib).max()) if ia.size else 0


@pytest.mark.parametrize("cols", [128, 1024, 160, 2880])
def test_rmsnorm_addnorm(ctx, cols):
    rng = np.random.default_rng(cols)
    rows = 3
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 3
    t = rng.standard_normal((rows, cols)).astype(np.float32)
    w = rng.standard_normal(cols).astype(np.float32)
    dx, dt, dw, dy = ctx.array(x), ctx.array(t), ctx.array(w), ctx.alloc(x.nbytes)
    H.check(H.lib().ihip_enqueue_rmsnorm(ctx.h, dx.ptr, dw.ptr, dy.ptr, rows, cols, 1e-6))
    got = dy.download(np.float32, x.size).reshape(x.shape)
    assert ulp(got, O.rmsnorm(x, w, 1e-6)) <= 1
    H.check(H.lib().ihip_enqueue_addnorm(ctx.h, dx.ptr, dt.ptr, dw.ptr, dy.ptr, rows, cols, 1e-5))
    xs = x + t
    assert np.array_equal(dx.download(np.float32, x.size).reshape(x.shape), xs)
    assert ulp(dy.download(np.float32, x.size).reshape(x.shape), O.rmsnorm(xs, w, 1e-5)) <= 1


@pytest.mark.parametrize("limit", [0.0, 7.0])
def test_swiglu(ctx, limit):
    rng = np.random.default_rng(3)
    n = 10000
    g = (rng.standard_normal(n) * 6).astype(np.float32)
    u = (rng.standard_normal(n) * 6).astype(np.float32)
    dg, du = ctx.array(g), ctx.array(u)
    H.check(H.lib().ihip_enqueue_swiglu(ctx.h, dg.ptr, du.ptr, n, 1.702, limit))
    got = dg.download(np.float32, n)
    ref = O.swiglu(g, u, 1.702 if limit else 1.0, limit)
    assert ulp(got, ref) <= 1


@pytest.mark.parametrize("hd,heads,kvh,norm,f16", [(128, 16, 8, True, False), (64, 64, 8, False, True)])
def test_qkrope_and_cache(ctx, hd, heads, kvh, norm, f16):
    rng = np.random.default_rng(hd)
    rows, past = 3, 5
    q = rng.standard_normal((rows, heads * hd)).astype(np.float32)
    k = rng.standard_normal((rows, kvh * hd)).astype(np.float32)
    v = rng.standard_normal((rows, kvh * hd)).astype(np.float32)
    qn = (rng.standard_normal(hd) * 0.1 + 1).astype(np.float32)
    kn = (rng.standard_normal(hd) * 0.1 + 1).astype(np.float32)
    ang = rng.uniform(0, 6.28, (rows, hd // 2)).astype(np.float32)
    cs = np.concatenate([np.cos(ang).ravel(), np.sin(ang).ravel()]).astype(np.float32)
    cache = (past + rows) * kvh * hd * (2 if f16 else 4)
    dq, dk, dv, dqn, dkn, dcs = (ctx.array(a) for a in (q, k, v, qn, kn, cs))
    dkc, dvc = ctx.alloc(cache), ctx.alloc(cache)
    H.check(H.lib().ihip_enqueue_qkrope(ctx.h, dq.ptr, dk.ptr, dv.ptr, dqn.ptr if norm else 0,
                                        dkn.ptr if norm else 0, dcs.ptr, dkc.ptr, dvc.ptr, rows,
                                        heads, kvh, hd, past, 1e-6, int(f16)))
    qr = O.rmsnorm(q.reshape(-1, hd), qn, 1e-6).reshape(q.shape) if norm else q
    kr = O.rmsnorm(k.reshape(-1, hd), kn, 1e-6).reshape(k.shape) if norm else k
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    qr = O.rope(qr, heads, hd, c, s)
    kr = O.rope(kr, kvh, hd, c, s)
    assert ulp(dq.download(np.float32, q.size).reshape(q.shape), qr) <= 1
    n = rows * kvh * hd
    off = past * kvh * hd
    if f16:
        kc = dkc.download(np.float16, off + n)[off:].astype(np.float32)
        vc = dvc.download(np.float16, off + n)[off:].astype(np.float32)
        assert np.array_equal(kc, kr.ravel().astype(np.float16).astype(np.float32)) or \
            ulp(kc, kr.ravel().astype(np.float16).astype(np.float32)) <= 1 << 13
        assert np.array_equal(vc, v.ravel().astype(np.float16).astype(np.float32))
    else:
        assert ulp(dkc.download(np.float32, off + n)[off:], kr.ravel()) <= 1
        assert np.array_equal(dvc.download(np.float32, off + n)[off:], v.ravel())


@pytest.mark.parametrize("hd,heads,kvh,past,rows,window,sinks,f16", [
    (128, 16, 8, 40, 1, 0, False, False),
    (128, 32, 4, 300, 3, 0, False, False),
    (64, 64, 8, 200, 2, 128, True, False),
    (64, 64, 8, 20, 5, 0, True, False),
    (128, 16, 8, 100, 1, 0, False, True),
    # tiles of 8 prompt rows: from position 0 (two ranges, the causal end
    # inside a tile), a window moving across a tile's rows, one whole tile,
    # a partial last tile under a window
    (128, 32, 4, 0, 130, 0, False, True),
    (64, 64, 8, 150, 20, 128, True, True),
    (128, 16, 8, 7, 8, 0, False, False),
    (64, 8, 2, 300, 33, 100, False, False),
    # tiles of 16 prompt rows on the f64 matrix cores: a whole tile, a
    # partial tile, three ranges from position 0, a window across tiles with
    # f16 keys and sinks, the largest tile key span (window start moving
    # inside a tile) with f32 keys
    (128, 32, 4, 0, 16, 0, True, False), (128, 16, 8, 5, 17, 0, False, False),
    (128, 32, 4, 0, 300, 0, True, True), (64, 64, 8, 300, 100, 128, True, True),
    (128, 8, 2, 500, 48, 200, False, False), (64, 8, 8, 40, 70, 0, False, True),
    # other head sizes (the ranges kernel): 24 (12 pairs in a 16-lane slot, the
    # tiny gpt-oss), 32, 96 and 192 (a second pair for half the lanes)
    (24, 4, 2, 10, 6, 5, True, True), (24, 4, 2, 150, 1, 0, True, False),
    (32, 4, 2, 200, 3, 0, False, True), (96, 8, 4, 130, 2, 0, False, False),
    (192, 4, 1, 60, 2, 0, True, True),
    # heads of 44 (no multiple of 8: keys read one value at a time), 320 and
    # 512 (Gemma 4's full layers: up to four pairs per lane)
    (44, 4, 1, 30, 3, 0, False, True), (44, 4, 2, 70, 2, 0, False, False),
    (320, 4, 2, 150, 2, 0, False, True), (512, 8, 1, 260, 3, 0, False, False),
    (512, 4, 2, 40, 1, 0, True, True),
    # heads of 256 (Qwen3.5, Gemma 4 sliding layers) with f16 keys: the paired
    # key scoring and the fused value sums, one row and a few
    (256, 8, 2, 300, 1, 0, True, True), (256, 16, 8, 1030, 1, 1024, True, False),
    (256, 4, 1, 90, 3, 0, True, False), (512, 16, 2, 700, 1, 0, True, False),
    (128, 32, 4, 1100, 1, 0, True, False),
    # one row whose keys fit one 128-key range: sinks with half-float keys,
    # a window with float keys and sinks, exactly 128 keys, a window of 128
    # past 128 keys (the decode step's own one-row kernel, which finishes
    # such a head in its range block, runs in the model tests: prompts of 12
    # and 16 tokens decode at most 128 keys)
    (64, 8, 2, 90, 1, 0, True, True), (128, 8, 2, 60, 1, 40, True, False),
    (128, 32, 4, 127, 1, 0, True, True), (64, 16, 4, 400, 1, 128, False, True)])
def test_attention(ctx, hd, heads, kvh, past, rows, window, sinks, f16):
    rng = np.random.default_rng(past + rows)
    T = past + rows
    q = rng.standard_normal((rows, heads * hd)).astype(np.float32)
    keys = rng.standard_normal((T, kvh * hd)).astype(np.float32)
    vals = rng.standard_normal((T, kvh * hd)).astype(np.float32)
    sk = rng.standard_normal(heads).astype(np.float32) * 2 if sinks else None
    if f16:
        keys = keys.astype(np.float16).astype(np.float32)
        vals = vals.astype(np.float16).astype(np.float32)
        dkc, dvc = ctx.array(keys.astype(np.float16)), ctx.array(vals.astype(np.float16))
    else:
        dkc, dvc = ctx.array(keys), ctx.array(vals)
    dq = ctx.array(q)
    dy = ctx.alloc(q.nbytes)
    ds = ctx.array(sk) if sinks else None
    H.check(H.lib().ihip_enqueue_attention(ctx.h, dq.ptr, dkc.ptr, dvc.ptr, dy.ptr, rows, heads,
                                           kvh, hd, past, window, ds.ptr if sinks else 0, 0.0,
                                           int(f16)))
    got = dy.download(np.float32, q.size).reshape(q.shape)
    ref = O.causal_attention(q, heads, hd, keys, vals, past, kvh, window, sk)
    assert ulp(got, ref) <= 2


@pytest.fixture(scope="module")
def ctx_rows():
    """A context whose prompt attention runs the VALU tiles of 8 rows
    (IHIP_ATTN_MFMA=0, read when the context is created)."""
    import os
    old = os.environ.get("IHIP_ATTN_MFMA")
    os.environ["IHIP_ATTN_MFMA"] = "0"
    try:
        c = H.Context(0)
    finally:
        if old is None:
            del os.environ["IHIP_ATTN_MFMA"]
        else:
            os.environ["IHIP_ATTN_MFMA"] = old
    yield c
    c.close()


@pytest.mark.parametrize("hd,heads,kvh,past,rows,window,sinks,f16", [
    (128, 32, 4, 0, 130, 0, False, True), (64, 64, 8, 150, 20, 128, True, True),
    (128, 16, 8, 7, 8, 0, False, False), (64, 8, 2, 300, 33, 100, False, False)])
def test_attention_valu_tiles(ctx_rows, hd, heads, kvh, past, rows, window, sinks, f16):
    """The VALU prompt tiles (kept as the IHIP_ATTN_MFMA=0 path) against the oracle."""
    test_attention(ctx_rows, hd, heads, kvh, past, rows, window, sinks, f16)


@pytest.mark.parametrize("E,k,norm,scaled", [(128, 8, True, False), (32, 4, True, False),
                                             (16, 3, False, False), (128, 8, True, True)])
def test_route(ctx, E, k, norm, scaled):
    rng = np.random.default_rng(E)
    sc = rng.uniform(0.5, 1.5, E).astype(np.float32) if scaled else None
    ds = ctx.array(sc) if scaled else None
    for trial in range(5):
        lg = rng.standard_normal(E).astype(np.float32)
        if trial == 1:
            lg[3] = lg[7] = lg.max() + 1  # a tie: the lower id first
        dl = ctx.array(lg)
        di, dw = ctx.alloc(4 * k), ctx.alloc(4 * k)
        H.check(H.lib().ihip_enqueue_route(ctx.h, dl.ptr, E, k, int(norm), di.ptr, dw.ptr,
                                           ds.ptr if scaled else 0))
        ids, w = O.route(lg, k, norm)
        if scaled:
            # Route's expert scale (decoder.pas:2939-2941): after the renorm
            w = (w * sc[ids]).astype(np.float32)
        order = np.argsort(ids, kind="stable")
        assert np.array_equal(di.download(np.int32, k), ids[order])
        assert np.array_equal(dw.download(np.float32, k), w[order])


def test_moecombine_and_argmax(ctx):
    rng = np.random.default_rng(1)
    k, n = 8, 2048
    d = rng.standard_normal((k, n)).astype(np.float32)
    w = rng.random(k).astype(np.float32)
    dd, dw, dy = ctx.array(d), ctx.array(w), ctx.alloc(n * 4)
    H.check(H.lib().ihip_enqueue_moecombine(ctx.h, dd.ptr, dw.ptr, dy.ptr, k, n))
    ref = np.zeros(n, np.float32)
    for s in range(k):
        ref = (ref + (w[s] * d[s]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(dy.download(np.float32, n), ref)
    for case in range(8):
        v = rng.standard_normal(151936).astype(np.float32)
        if case == 1:
            v[[5, 70000]] = v.max() + 1  # tie: the first index
        if case == 2:
            v[::3] = np.nan
        if case == 3:
            v[:] = np.nan
        if case == 4:  # -0 before +0 at the top: equal keys, the first index
            v = -np.abs(v) - 1
            v[[77, 150000]] = [-0.0, 0.0]
        if case == 5:  # one value; a short row
            v = v[:1]
        if case == 6:
            v = v[:1000]
        if case == 7:  # -inf everywhere but a NaN and +inf at the end
            v[:] = -np.inf
            v[-2:] = [np.nan, np.inf]
        dv, do = ctx.array(v), ctx.alloc(4)
        H.check(H.lib().ihip_enqueue_argmax(ctx.h, dv.ptr, v.size, do.ptr))
        assert int(do.download(np.int32, 1)[0]) == O.argmax(v)
