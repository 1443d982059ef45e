"""The CPU oracle pinned against the reference's golden vectors
(tests/data/infer-ref/{q8,q4,q5,q51,qk,mxfp4,ops} of the reference, copied as
data into tests/golden/): the checks of tests/test.infer.gguf.pas:275-809
(HalfFloatLikeGgml, QuantizeLikeGgml, LinearQ8LikeGgml, Q4LikeGgml,
Q5LikeGgml, Q51LikeGgml, Mxfp4LikeGgml, KQuantsLikeGgml), with the
reference's tolerances."""
import numpy as np
import pytest

import oracle_lib as O
from golden_io import GoldenSet, compare


def test_half_like_ggml():
    g = GoldenSet("q8")
    x, bits = g["half/x"], g["half/bits"]
    mine = np.array([O.lib().orc_single_to_half(float(v)) for v in x], np.int64)
    assert np.array_equal(mine, bits.astype(np.int64) & 0xFFFF)


def test_half_to_single_all_patterns():
    # every half pattern against numpy's IEEE widening (NaN: sign and payload
    # kept, the bits the reference writes - tensor.pas:319)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32).view(np.uint32)
    mine = np.array([O.lib().orc_half_to_single_bits(int(v)) for v in h], np.uint32)
    nan = np.isnan(h.view(np.float16))
    assert np.array_equal(mine[~nan], ref[~nan])
    # NaN: exponent all ones, mantissa shifted in unchanged
    exp_nan = (0x7F800000 | ((h[nan].astype(np.uint32) & 0x3FF) << 13)
               | ((h[nan].astype(np.uint32) & 0x8000) << 16))
    assert np.array_equal(mine[nan], exp_nan)


def test_single_to_half_roundtrip_and_rne():
    # every finite half survives single -> half; midpoints round to even
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16)
    fin = np.isfinite(f)
    back = np.array([O.lib().orc_single_to_half(float(v)) for v in f[fin].astype(np.float32)])
    assert np.array_equal(back.astype(np.uint16), h[fin])
    rng = np.random.default_rng(1)
    xs = rng.standard_normal(20000).astype(np.float32) * np.float32(2.0) ** rng.integers(
        -30, 17, 20000).astype(np.float32)
    mine = np.array([O.lib().orc_single_to_half(float(v)) for v in xs], np.uint16)
    assert np.array_equal(mine, xs.astype(np.float16).view(np.uint16))


def test_e8m0():
    for e in range(256):
        b = O.lib().orc_e8m0_half_bits(e)
        v = np.array([b], np.uint32).view(np.float32)[0]
        assert v == np.float32(2.0 ** (e - 128)) or (e == 255 and v == np.float32(2.0 ** 127))


@pytest.mark.parametrize("name,ties_away", [("q8", False), ("q4", True)])
def test_quantize_q8_0_like_ggml(name, ties_away):
    g = GoldenSet(name)
    key = "quant" if name == "q8" else "q8ref"
    x, blocks = g[f"{key}/x"], g[f"{key}/blocks"]
    for r in range(x.shape[0]):
        mine, bad = O.quantize_q8_0(x[r], ties_away)
        assert bad == 0
        assert np.array_equal(mine, blocks[r]), f"row {r}"


def test_quantize_q8_0_refuses_nonfinite():
    for r in range(4):
        bad = np.zeros(32, np.float32)
        if r < 2:
            bad.view(np.uint32)[5 + r * 20] = 0x7FC00000
        else:
            bad.view(np.uint32)[r] = 0x7F800000 | ((r & 1) << 31)
        bad[0] = 1
        _, b = O.quantize_q8_0(bad)
        assert b != 0


def test_quantize_q4_0_like_ggml():
    g = GoldenSet("q4")
    x, blocks = g["quant/x"], g["quant/blocks"]
    for r in range(x.shape[0]):
        mine, bad = O.quantize_q4_0(x[r])
        assert bad == 0 and np.array_equal(mine, blocks[r]), f"row {r}"


def test_quantize_q8_k_like_ggml():
    g = GoldenSet("qk")
    x, blocks = g["q8k/x"], g["q8k/blocks"]
    for r in range(x.shape[0]):
        mine, bad = O.quantize_q8_k(x[r])
        assert bad == 0 and np.array_equal(mine, blocks[r]), f"row {r}"


DEQUANT = [("q8", "linear/weight", "dequant/y", O.Q8_0), ("q4", "quant/blocks", "dequant/y", O.Q4_0),
           ("q5", "quant/blocks", "dequant/y", O.Q5_0), ("q51", "quant/blocks", "dequant/y", O.Q5_1),
           ("mxfp4", "quant/blocks", "dequant/y", O.MXFP4),
           ("qk", "q4_K/weight", "q4_K/dequant", O.Q4_K), ("qk", "q6_K/weight", "q6_K/dequant", O.Q6_K)]


@pytest.mark.parametrize("name,wkey,ykey,dtype", DEQUANT)
def test_dequant_exact(name, wkey, ykey, dtype):
    g = GoldenSet(name)
    w, y = g[wkey], g[ykey]
    rows, cols = y.shape
    mine = O.dequant(np.ascontiguousarray(w), dtype, rows, cols)
    assert np.array_equal(mine.view(np.uint32), y.view(np.uint32))


LINEAR = [("q8", "linear/weight", "linear/y", O.Q8_0, 1e-5, 1e-5),
          ("q4", "linear/weight", "linear/y", O.Q4_0, 1e-5, 1e-5),
          ("q5", "linear/weight", "linear/y", O.Q5_0, 1e-5, 1e-5),
          ("q51", "linear/weight", "linear/y", O.Q5_1, 2e-3, 2e-4),
          ("mxfp4", "linear/weight", "linear/y", O.MXFP4, 1e-5, 1e-5),
          ("qk", "q4_K/weight", "q4_K/y", O.Q4_K, 1e-4, 1e-5),
          ("qk", "q6_K/weight", "q6_K/y", O.Q6_K, 1e-4, 1e-5)]


@pytest.mark.parametrize("name,wkey,ykey,dtype,atol,rtol", LINEAR)
def test_linear_like_ggml(name, wkey, ykey, dtype, atol, rtol):
    g = GoldenSet(name)
    x, b, w, y = g["linear/x"], g["linear/bias"], g[wkey], g[ykey]
    mine = O.linear(x, np.ascontiguousarray(w), dtype, b.size, b)
    ok, err = compare(mine, y, atol, rtol)
    assert ok, err


def test_linear_f32_ops_fixture():
    g = GoldenSet("ops")
    x, w, b, y = g["linear/x"], g["linear/weight"], g["linear/bias"], g["linear/y"]
    mine = O.linear(x, np.ascontiguousarray(w), O.F32, b.size, b)
    assert np.array_equal(mine, y)  # double sums, one rounding: the fixture's bits
    mine = O.linear(x, np.ascontiguousarray(w), O.F32, b.size, b, f32=True)
    assert np.array_equal(mine, y)


def test_mxfp4_edge_exponents_exact():
    # test.infer.cuda.pas:840-864: exponents {0, 1, 2, 127, 128, 200}, x = 1,
    # every nibble: the dequantized values are powers of two times k
    ks = [0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12]
    for e in (0, 1, 2, 127, 128, 200, 253, 254, 255):
        blk = np.zeros(17, np.uint8)
        blk[0] = e
        blk[1:] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
        y = O.dequant(blk, O.MXFP4, 1, 32)[0]
        with np.errstate(over="ignore"):
            want = np.array([np.float32(2.0 ** (e - 128)) * np.float32(k) for k in
                             [ks[j] for j in range(16)] + [ks[15 - j] for j in range(16)]],
                            np.float32)
        assert np.array_equal(y, want), e
