"""ctypes binding of oracle/liboracle.so - the CPU checker (test
infrastructure only: the product never loads it)."""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "liboracle.so")

F32, F16, BF16, Q8_0, Q4_0, Q4_K, Q6_K, Q5_0, MXFP4, Q5_1 = 1, 2, 3, 8, 9, 10, 11, 12, 13, 14
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q4_0: (32, 18),
         Q4_K: (256, 144), Q6_K: (256, 210), Q5_0: (32, 22), MXFP4: (32, 17), Q5_1: (32, 24)}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            import subprocess
            subprocess.check_call(["make", "-s", "-C", os.path.dirname(LIB_PATH)])
        L = C.CDLL(LIB_PATH)
        vp, i64, f32p = C.c_void_p, C.c_int64, C.POINTER(C.c_float)
        L.orc_half_to_single_bits.restype = C.c_uint32
        L.orc_half_to_single_bits.argtypes = [C.c_uint16]
        L.orc_single_to_half.restype = C.c_uint16
        L.orc_single_to_half.argtypes = [C.c_float]
        L.orc_e8m0_half_bits.restype = C.c_uint32
        L.orc_e8m0_half_bits.argtypes = [C.c_uint8]
        L.orc_row_to_f32.argtypes = [vp, C.c_int, i64, i64, vp]
        for n in ("orc_quantize_q4_0", "orc_quantize_q8_k"):
            getattr(L, n).restype = i64
            getattr(L, n).argtypes = [vp, i64, vp]
        L.orc_quantize_q8_0.restype = i64
        L.orc_quantize_q8_0.argtypes = [vp, i64, vp, C.c_int]
        for n in ("orc_linear", "orc_linear_f32"):
            getattr(L, n).argtypes = [vp, i64, i64, vp, C.c_int, i64, vp, vp, C.c_int]
        L.orc_rmsnorm.argtypes = [vp, i64, i64, vp, C.c_double, vp]
        L.orc_rmsnorm.restype = None
        L.orc_swiglu.argtypes = [vp, vp, i64, C.c_float, C.c_float]
        L.orc_swiglu.restype = None
        L.orc_rope.argtypes = [vp, i64, i64, i64, vp, vp, i64]
        L.orc_rope.restype = None
        L.orc_causal_attention.argtypes = [vp, i64, i64, i64, vp, vp, i64, i64, vp, i64, vp,
                                           C.c_double]
        L.orc_causal_attention.restype = None
        L.orc_route.argtypes = [vp, i64, i64, C.c_int, vp, vp]
        L.orc_route.restype = None
        L.orc_argmax.restype = i64
        L.orc_argmax.argtypes = [vp, i64]
        L.orc_rotary.argtypes = [vp, i64, i64, vp]
        L.orc_rotary2.argtypes = [vp, i64, i64, i64, vp]
        L.orc_geglu.argtypes = [vp, vp, i64]
        L.orc_geglu.restype = None
        L.orc_softcap.argtypes = [vp, i64, C.c_double]
        L.orc_softcap.restype = None
        L.orc_gate_sigmoid.argtypes = [vp, vp, i64]
        L.orc_gate_sigmoid.restype = None
        L.orc_delta_prep.argtypes = [vp, vp, vp, vp, i64, vp, vp, vp, vp, i64, i64, i64, i64, i64]
        L.orc_delta_prep.restype = None
        L.orc_delta_rule.argtypes = [vp, i64, i64, i64, i64, i64, i64, i64, vp, vp, vp, vp]
        L.orc_delta_rule.restype = None
        L.orc_model_create.argtypes = [vp, i64, C.c_int, C.c_int, C.POINTER(vp)]
        L.orc_model_destroy.argtypes = [vp]
        L.orc_model_destroy.restype = None
        L.orc_model_set_f32.argtypes = [vp, C.c_int]
        L.orc_model_set_f32.restype = None
        L.orc_model_forward_rows.argtypes = [vp, vp, vp, i64, vp, C.c_int, vp]
        L.orc_model_truncate.argtypes = [vp, i64]
        L.orc_model_set_threads.argtypes = [vp, C.c_int]
        L.orc_model_set_threads.restype = None
        L.orc_model_set_fast.argtypes = [vp, C.c_int]
        L.orc_model_set_fast.restype = None
        L.orc_fast_available.restype = C.c_int
        L.orc_fast_linear.argtypes = [vp, i64, i64, vp, C.c_int, i64, vp, vp, C.c_int]
        L.orc_fast_attention.argtypes = [vp, i64, i64, i64, vp, vp, i64, i64, vp, i64, vp,
                                         C.c_int]
        L.orc_fast_attention.restype = None
        L.orc_model_route_gap.restype = C.c_double
        L.orc_model_route_gap.argtypes = [vp]
        L.orc_model_route_record.argtypes = [vp, vp, vp, i64]
        L.orc_model_route_record.restype = None
        L.orc_model_route_recorded.argtypes = [vp]
        L.orc_model_route_recorded.restype = i64
        L.orc_model_forward.argtypes = [vp, vp, i64, vp, C.c_int]
        L.orc_model_greedy.argtypes = [vp, vp, i64, i64, vp, vp]
        L.orc_splitmix_next.restype = C.c_double
        L.orc_splitmix_next.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_sampler_create.argtypes = [C.c_double, C.c_int32, C.c_double, C.c_double,
                                         C.c_int64, C.POINTER(vp)]
        L.orc_sampler_destroy.argtypes = [vp]
        L.orc_sampler_destroy.restype = None
        L.orc_sampler_next.restype = i64
        L.orc_sampler_next.argtypes = [vp, vp, i64]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def row_bytes(dtype, cols):
    bv, bs = BLOCK[dtype]
    return cols // bv * bs


def dequant(w, dtype, rows, cols):
    out = np.empty((rows, cols), np.float32)
    for r in range(rows):
        assert lib().orc_row_to_f32(_p(w), dtype, r, cols, out[r].ctypes.data) == 0
    return out


def quantize_q8_0(x, ties_away=False):
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(x.size // 32 * 34, np.uint8)
    bad = lib().orc_quantize_q8_0(_p(x), x.size, _p(out), int(ties_away))
    return out, bad


def quantize_q4_0(x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(x.size // 32 * 18, np.uint8)
    bad = lib().orc_quantize_q4_0(_p(x), x.size, _p(out))
    return out, bad


def quantize_q8_k(x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(x.size // 256 * 292, np.uint8)
    bad = lib().orc_quantize_q8_k(_p(x), x.size, _p(out))
    return out, bad


def linear(x, w, dtype, out, bias=None, threads=8, f32=False):
    x = np.ascontiguousarray(x, np.float32)
    rows, nin = x.shape
    y = np.empty((rows, out), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    fn = lib().orc_linear_f32 if f32 else lib().orc_linear
    rc = fn(_p(x), rows, nin, _p(w), dtype, out, _p(b), _p(y), threads)
    if rc:
        raise ValueError(f"oracle linear failed: {rc}")
    return y


def fast_available():
    return bool(lib().orc_fast_available())


def fast_linear(x, w, dtype, out, bias=None, threads=8):
    """TInferCpuFastBackend.Linear's default mode (AVX2, tiles of 16)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, nin = x.shape
    y = np.empty((rows, out), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    rc = lib().orc_fast_linear(_p(x), rows, nin, _p(w), dtype, out, _p(b), _p(y), threads)
    if rc:
        raise ValueError(f"fast linear failed: {rc}")
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), x.shape[0], x.shape[1], _p(np.ascontiguousarray(w, np.float32)),
                      eps, _p(y))
    return y


def swiglu(g, u, alpha=1.0, limit=0.0):
    g = np.array(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    lib().orc_swiglu(_p(g), _p(u), g.size, alpha, limit)
    return g


def rope(x, heads, hd, cos, sin, rot=0):
    x = np.array(x, np.float32)
    lib().orc_rope(_p(x), x.shape[0], heads, hd, _p(np.ascontiguousarray(cos, np.float32)),
                   _p(np.ascontiguousarray(sin, np.float32)), rot)
    return x


def causal_attention(q, heads, hd, keys, values, past, kvh, window=0, sinks=None, scale=0.0):
    q = np.ascontiguousarray(q, np.float32)
    y = np.empty_like(q)
    s = None if sinks is None else np.ascontiguousarray(sinks, np.float32)
    lib().orc_causal_attention(_p(q), q.shape[0], heads, hd,
                               _p(np.ascontiguousarray(keys, np.float32)),
                               _p(np.ascontiguousarray(values, np.float32)),
                               past, kvh, _p(y), window, _p(s), scale)
    return y


def route(logits, k, norm_topk=True):
    lg = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().orc_route(_p(lg), lg.size, k, int(norm_topk), _p(ids), _p(w))
    return ids, w


def geglu(g, u):
    """GeluTanhGlu: gelu_tanh(g) * u."""
    g = np.array(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    lib().orc_geglu(_p(g), _p(u), g.size)
    return g


def softcap(x, cap):
    x = np.array(x, np.float32)
    lib().orc_softcap(_p(x), x.size, float(cap))
    return x


def rotary2(desc, hd2, first, rows):
    """Rotary2: ([rows, hd2 / 2] cos, sin) of the second set."""
    cs = np.empty(rows * hd2, np.float32)
    lib().orc_rotary2(C.addressof(desc.struct), hd2, first, rows, _p(cs))
    half = hd2 // 2
    return cs[:rows * half].reshape(rows, half), cs[rows * half:].reshape(rows, half)


def gate_sigmoid(a, gate):
    """GateBySigmoid: a * sigmoid(gate)."""
    a = np.array(a, np.float32)
    g = np.ascontiguousarray(gate, np.float32)
    lib().orc_gate_sigmoid(_p(a), _p(g), a.size)
    return a


def delta_prep(qkv, beta, decay, z, conv, conv_w, dt_bias, neg_a, kh, vh, dk, dv, kw):
    """DeltaPrep over rows: returns (qkv, beta, decay, z, conv) after it."""
    out = [np.array(v, np.float32) for v in (qkv, beta, decay, z, conv)]
    w = [np.ascontiguousarray(v, np.float32) for v in (conv_w, dt_bias, neg_a)]
    lib().orc_delta_prep(_p(out[0]), _p(out[1]), _p(out[2]), _p(out[3]), out[0].shape[0],
                         _p(out[4]), _p(w[0]), _p(w[1]), _p(w[2]), kh, vh, dk, dv, kw)
    return out


def delta_rule(qkv, kh, vh, dk, dv, group, beta, decay, state):
    """DeltaRule (double branch): returns (y [rows, vh * dv], state after)."""
    q = np.ascontiguousarray(qkv, np.float32)
    st = np.array(state, np.float32)
    y = np.zeros((q.shape[0], vh * dv), np.float32)
    b = np.ascontiguousarray(beta, np.float32)
    g = np.ascontiguousarray(decay, np.float32)
    lib().orc_delta_rule(_p(q), q.shape[0], q.shape[1], kh, vh, dk, dv, group, _p(b), _p(g),
                         _p(st), _p(y))
    return y, st


class Sampler:
    """TInferSampler (sampler.pas:52-435) on the CPU: temperature, top_k,
    top_p, min_p, seed."""

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=0):
        self.h = None
        h = C.c_void_p()
        rc = lib().orc_sampler_create(temperature, top_k, top_p, min_p, seed, C.byref(h))
        if rc:
            raise ValueError("sampling settings out of range")
        self.h = h

    def next(self, logits):
        v = np.ascontiguousarray(logits, np.float32)
        return int(lib().orc_sampler_next(self.h, _p(v), v.size))

    def close(self):
        if self.h:
            lib().orc_sampler_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


def argmax(v):
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().orc_argmax(_p(v), v.size))


class Model:
    """The CPU decoder over a model description (mormot_ai_hip.ihip_model_desc)."""

    def __init__(self, desc, max_tokens, kv_f16=False, threads=None, f32=False, fast=False):
        self.desc = desc  # keeps the host tensors alive
        if threads is None:
            # a tiny model's Linear is too short for a thread pool (and the
            # test workers already share the cores)
            threads = 1 if desc.struct.hidden <= 512 else 8
        h = C.c_void_p()
        rc = lib().orc_model_create(C.addressof(desc.struct), max_tokens, int(kv_f16), threads,
                                    C.byref(h))
        if rc:
            raise RuntimeError(rc)
        self.h = h
        if f32:
            lib().orc_model_set_f32(self.h, 1)
        if fast:
            lib().orc_model_set_fast(self.h, 1)

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def forward(self, ids, all_logits=False):
        ids = np.ascontiguousarray(ids, np.int32)
        V = self.desc.vocab
        lg = np.empty((len(ids) if all_logits else 1, V), np.float32)
        rc = lib().orc_model_forward(self.h, _p(ids), len(ids), _p(lg), int(all_logits))
        if rc:
            raise RuntimeError(rc)
        return lg if all_logits else lg[0]

    def forward_embeds(self, embeds, hidden, normed=False):
        """ForwardEmbeds: (last row's logits, its final norm or None)."""
        e = np.ascontiguousarray(embeds, np.float32).reshape(-1, hidden)
        lg = np.empty(self.desc.vocab, np.float32)
        nv = np.empty(hidden, np.float32) if normed else None
        rc = lib().orc_model_forward_rows(self.h, None, _p(e), e.shape[0], _p(lg), 0, _p(nv))
        if rc:
            raise RuntimeError(rc)
        return lg, nv

    def truncate(self, length):
        if lib().orc_model_truncate(self.h, int(length)):
            raise ValueError("truncate beyond the cached tokens")

    def set_threads(self, n):
        lib().orc_model_set_threads(self.h, int(n))

    def route_gap(self):
        """The smallest k-th vs (k+1)-th router logit gap of the rows routed
        since the last call (inf for a dense model)."""
        return float(lib().orc_model_route_gap(self.h))

    def record_routes(self, rows, k):
        """TDecoderRouteTape in record mode: keep the picks (by id) and
        weights of up to `rows` routed rows from now on; routes() returns
        those recorded so far."""
        self._rec = (np.zeros((rows, k), np.int32), np.zeros((rows, k), np.float32))
        lib().orc_model_route_record(self.h, _p(self._rec[0]), _p(self._rec[1]), rows)

    def routes(self):
        n = int(lib().orc_model_route_recorded(self.h))
        return self._rec[0][:n].copy(), self._rec[1][:n].copy()

    def greedy(self, prompt, max_new):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max_new, np.int32)
        margins = np.empty(max_new, np.float32)
        rc = lib().orc_model_greedy(self.h, _p(p), len(p), max_new, _p(out), _p(margins))
        if rc:
            raise RuntimeError(rc)
        return out, margins
