"""ihip_enqueue_linear_at_static (the Linear that allocates nothing: its
quantized activations in a fixed device array) against
ihip_enqueue_linear_at on the same inputs, through the C-ABI: bit-equal
outputs on two calls in a row, the second with fewer rows (the array keeps
the first call's bytes), on both sides of the GEMM threshold, and the
refusal of a call that would not fit, and of a multi-row call of a second
context on the same GPU while the first holds the array."""
import ctypes as C

import numpy as np
import pytest

import infer_hip as H

pytestmark = pytest.mark.gpu


# a context per test: the first context of a device to make a multi-row call
# holds the array until it is destroyed
@pytest.fixture()
def ctx():
    c = H.Context(0)
    yield c
    c.close()


def run(ctx, fn, x, w_dev, dtype, out, bias_dev, mode):
    rows, nin = x.shape
    xb = H.Buffer(ctx, x.nbytes)
    xb.upload(x)
    yb = H.Buffer(ctx, rows * out * 4)
    H.check(fn(ctx.h, xb.ptr, rows, nin, dtype, w_dev, out, yb.ptr, bias_dev, mode), fn.__name__)
    H.check(H.lib().ihip_synchronize(ctx.h), "sync")
    y = yb.download(np.float32, rows * out).reshape(rows, out)
    xb.free()
    yb.free()
    return y


@pytest.mark.parametrize("dtype", [H.Q8_0, H.Q4_K, H.MXFP4, H.Q6_K])
@pytest.mark.parametrize("mode", [H.MODE_Q8, H.MODE_F32])
def test_static_matches_allocating_entry_point(ctx, dtype, mode):
    nin, out = 2048, 384
    w = H.synth_normal(dtype, out, nin, 77, 0.05)
    wd = C.c_uint64()
    H.check(H.lib().ihip_weight(ctx.h, H._p(w), dtype, out, nin, 1, C.byref(wd)), "weight")
    bias = np.random.default_rng(3).standard_normal(out).astype(np.float32)
    bd = C.c_uint64()
    H.check(H.lib().ihip_weight_f32(ctx.h, H._p(bias), out, C.byref(bd)), "bias")
    rng = np.random.default_rng(dtype * 10 + mode)
    # 200 rows (the MFMA GEMM), then 40 rows (8-row GEMVs), then one row
    for rows in (200, 40, 1):
        x = rng.standard_normal((rows, nin)).astype(np.float32)
        a = run(ctx, H.lib().ihip_enqueue_linear_at_static, x, wd.value, dtype, out, bd.value, mode)
        b = run(ctx, H.lib().ihip_enqueue_linear_at, x, wd.value, dtype, out, bd.value, mode)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rows, np.abs(a - b).max())
    # the cache is keyed by host address: forget both before the arrays go
    for a in (w, bias):
        assert H.lib().ihip_forget_weights(ctx.h, H._p(a), C.c_void_p(a.ctypes.data + a.nbytes)) >= 0


def test_static_refuses_beyond_its_size(ctx):
    nin, out, dtype = 4096, 64, H.Q8_0
    rows = (8 << 20) // (nin + nin // 8) + 1  # one row more than the array holds
    w = H.synth_normal(dtype, out, nin, 5, 0.05)
    wd = C.c_uint64()
    H.check(H.lib().ihip_weight(ctx.h, H._p(w), dtype, out, nin, 1, C.byref(wd)), "weight")
    xb = H.Buffer(ctx, rows * nin * 4)
    yb = H.Buffer(ctx, rows * out * 4)
    rc = H.lib().ihip_enqueue_linear_at_static(ctx.h, xb.ptr, rows, nin, dtype, wd.value, out,
                                               yb.ptr, 0, H.MODE_Q8)
    assert rc == H.IHIP_E_NOMEM
    assert b"static scratch" in H.lib().ihip_last_error()
    assert H.lib().ihip_forget_weights(ctx.h, H._p(w), C.c_void_p(w.ctypes.data + w.nbytes)) >= 0
    H.check(H.lib().ihip_synchronize(ctx.h), "sync")
    xb.free()
    yb.free()


def test_static_refuses_a_second_context():
    """The array belongs to the first context of a device that makes a
    multi-row call, until it is destroyed: a second context's multi-row call
    is refused (their streams are not ordered), its one-row call is not."""
    nin, out, dtype = 1024, 128, H.Q8_0
    w = H.synth_normal(dtype, out, nin, 9, 0.05)
    x = np.random.default_rng(4).standard_normal((16, nin)).astype(np.float32)
    a, b = H.Context(0), H.Context(0)
    try:
        wa, wb = C.c_uint64(), C.c_uint64()
        H.check(H.lib().ihip_weight(a.h, H._p(w), dtype, out, nin, 1, C.byref(wa)), "weight")
        H.check(H.lib().ihip_weight(b.h, H._p(w), dtype, out, nin, 1, C.byref(wb)), "weight")
        static = H.lib().ihip_enqueue_linear_at_static
        ya = run(a, static, x, wa.value, dtype, out, 0, H.MODE_Q8)
        xb = H.Buffer(b, x.nbytes)
        yb = H.Buffer(b, 16 * out * 4)
        rc = static(b.h, xb.ptr, 16, nin, dtype, wb.value, out, yb.ptr, 0, H.MODE_Q8)
        assert rc == H.IHIP_E_ARG and b"another context" in H.lib().ihip_last_error()
        xb.free()
        yb.free()
        y1 = run(b, static, x[:1], wb.value, dtype, out, 0, H.MODE_Q8)
        assert np.array_equal(y1.view(np.uint32), ya[:1].view(np.uint32))
        # the holder destroyed: the other context may take the array
        H.lib().ihip_forget_weights(a.h, H._p(w), C.c_void_p(w.ctypes.data + w.nbytes))
        a.close()
        a = None
        yb2 = run(b, static, x, wb.value, dtype, out, 0, H.MODE_Q8)
        assert np.array_equal(yb2.view(np.uint32), ya.view(np.uint32))
        H.lib().ihip_forget_weights(b.h, H._p(w), C.c_void_p(w.ctypes.data + w.nbytes))
    finally:
        if a is not None:
            a.close()
        b.close()
