"""Python binding of libmormot_ai_hip.so (the C-ABI of include/mormot_ai_hip.h).

The binding the reference's Pascal host would declare as `external`
functions, restated with ctypes: the tests and bench.py drive the HIP backend
through exactly the entry points a Pascal unit binds. There is no fallback: a
missing library or device raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(HERE), "libmormot_ai_hip.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(HERE)), "include", "mormot_ai_hip.h")

# TInferDType ordinals
F32, F16, BF16, Q8_0, Q4_0, Q4_K, Q6_K, Q5_0, MXFP4, Q5_1 = 1, 2, 3, 8, 9, 10, 11, 12, 13, 14
NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q8_0: "Q8_0", Q4_0: "Q4_0", Q4_K: "Q4_K",
         Q6_K: "Q6_K", Q5_0: "Q5_0", MXFP4: "MXFP4", Q5_1: "Q5_1"}
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q4_0: (32, 18),
         Q4_K: (256, 144), Q6_K: (256, 210), Q5_0: (32, 22), MXFP4: (32, 17), Q5_1: (32, 24)}
MODE_F32, MODE_Q8 = 0, 1


class HipError(RuntimeError):
    pass


def row_bytes(dtype, cols):
    bv, bs = BLOCK[dtype]
    return cols // bv * bs


_lib = None


def lib():
    """The loaded library; raises when it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        vp, i64, u64, i32 = C.c_void_p, C.c_int64, C.c_uint64, C.c_int
        sig = {
            "ihip_available": (i32, []),
            "ihip_last_error": (C.c_char_p, []),
            "ihip_create": (i32, [i32, C.POINTER(vp)]),
            "ihip_destroy": (None, [vp]),
            "ihip_device_info": (i32, [vp, C.c_char_p, i32, C.POINTER(u64), C.POINTER(i32)]),
            "ihip_alloc": (i32, [vp, u64, C.POINTER(u64)]),
            "ihip_free": (i32, [vp, u64]),
            "ihip_upload": (i32, [vp, u64, vp, u64]),
            "ihip_download": (i32, [vp, vp, u64, u64]),
            "ihip_upload_async": (i32, [vp, u64, vp, u64]),
            "ihip_copy_async": (i32, [vp, u64, u64, u64]),
            "ihip_synchronize": (i32, [vp]),
            "ihip_capture_begin": (i32, [vp]),
            "ihip_capture_end": (i32, [vp, i32]),
            "ihip_graph_launch": (i32, [vp, i32]),
            "ihip_event_record": (i32, [vp, i32]),
            "ihip_event_elapsed": (i32, [vp, i32, i32, C.POINTER(C.c_float)]),
            "ihip_type_bytes": (u64, [i32, u64]),
            "ihip_weight": (i32, [vp, vp, i32, i64, i64, i64, C.POINTER(u64)]),
            "ihip_repack": (i32, [vp, vp, i32, i64, i64, i64, i32]),
            "ihip_weight_f32": (i32, [vp, vp, i64, C.POINTER(u64)]),
            "ihip_forget_weights": (i32, [vp, vp, vp]),
            "ihip_clear_weights": (i32, [vp]),
            "ihip_gpu_linear": (i32, [i32, i64]),
            "ihip_enqueue_linear_at": (i32, [vp, u64, i64, i64, i32, u64, i64, u64, u64, i32]),
            "ihip_enqueue_linear_ids": (i32, [vp, u64, i64, i32, u64, i64, i64, u64, i64, i32,
                                              u64, u64, i32]),
            "ihip_linear": (i32, [vp, vp, i64, i64, vp, i32, i64, vp, vp, i32]),
            "ihip_enqueue_dequant": (i32, [vp, u64, i32, i64, i64, i64, i64, u64]),
            "ihip_q8_bytes": (u64, [i64, i32]),
            "ihip_enqueue_quantize": (i32, [vp, u64, i64, i64, i32, u64, u64]),
            "ihip_enqueue_rmsnorm": (i32, [vp, u64, u64, u64, i64, i64, C.c_double]),
            "ihip_enqueue_addnorm": (i32, [vp, u64, u64, u64, u64, i64, i64, C.c_double]),
            "ihip_enqueue_add": (i32, [vp, u64, u64, i64]),
            "ihip_enqueue_swiglu": (i32, [vp, u64, u64, i64, C.c_float, C.c_float]),
            "ihip_enqueue_qkrope": (i32, [vp, u64, u64, u64, u64, u64, u64, u64, u64, i64, i64,
                                          i64, i64, i64, C.c_double, i32]),
            "ihip_enqueue_attention": (i32, [vp, u64, u64, u64, u64, i64, i64, i64, i64, i64, i64,
                                             u64, C.c_double, i32]),
            "ihip_enqueue_route": (i32, [vp, u64, i64, i64, i32, u64, u64]),
            "ihip_enqueue_moecombine": (i32, [vp, u64, u64, u64, i64, i64]),
            "ihip_enqueue_embed": (i32, [vp, u64, i32, i64, i64, u64, i64, u64]),
            "ihip_enqueue_argmax": (i32, [vp, u64, i64, u64]),
            "ihip_model_create": (i32, [vp, vp, i32, i32, i64, C.POINTER(vp)]),
            "ihip_model_destroy": (None, [vp]),
            "ihip_model_reset": (i32, [vp]),
            "ihip_model_forward": (i32, [vp, vp, i64, vp, i32]),
            "ihip_model_greedy": (i32, [vp, vp, i64, i64, vp]),
            "ihip_model_decode": (i32, [vp, C.c_int32, i64, vp]),
            "ihip_model_use_graphs": (i32, [vp, i32]),
            "ihip_model_chunk": (i32, [vp, i64]),
            "ihip_enqueue_stream_read": (i32, [vp, u64, u64, u64]),
            "ihip_model_rotary": (i32, [vp, i64, i64, vp]),
            "ihip_model_timing": (i32, [vp, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
            "ihip_synth_blocks": (i32, [vp, i32, i64, i64, u64, i32, i32, i32]),
            "ihip_synth_normal": (i32, [vp, i32, i64, i64, u64, C.c_float, i32]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def header_symbols():
    """Every function include/mormot_ai_hip.h declares."""
    import re
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ihip_[a-z0-9_]+)\s*\(", text)))


def check(rc, what=""):
    if rc != 0:
        msg = lib().ihip_last_error().decode(errors="replace")
        raise HipError(f"{what}: status {rc}: {msg}")


def _p(a):
    return None if a is None else a.ctypes.data


def available():
    return lib().ihip_available()


def synth_blocks(dtype, rows, cols, seed, lo=-8, hi=-4, threads=0):
    out = np.empty(rows * row_bytes(dtype, cols), np.uint8)
    check(lib().ihip_synth_blocks(_p(out), dtype, rows, cols, seed, lo, hi, threads), "synth")
    return out


def synth_normal(dtype, rows, cols, seed, sigma=0.02, threads=0):
    out = np.empty(rows * row_bytes(dtype, cols), np.uint8)
    check(lib().ihip_synth_normal(_p(out), dtype, rows, cols, seed, sigma, threads), "synth")
    return out


def repack(src, dtype, out, cols, count=1, inverse=False):
    dst = np.empty_like(src)
    check(lib().ihip_repack(_p(src), _p(dst), dtype, out, cols, count, int(inverse)), "repack")
    return dst


class Buffer:
    """A device buffer (TInferCuBuffer)."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        d = C.c_uint64()
        check(lib().ihip_alloc(ctx.h, self.nbytes, C.byref(d)), "alloc")
        self.ptr = d.value

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().ihip_upload(self.ctx.h, self.ptr, _p(a), a.nbytes), "upload")

    def download(self, dtype, count):
        out = np.empty(count, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().ihip_download(self.ctx.h, _p(out), self.ptr, out.nbytes), "download")
        return out

    def free(self):
        if self.ptr:
            check(lib().ihip_free(self.ctx.h, self.ptr), "free")
            self.ptr = 0


class Context:
    """One device and stream (TInferCuda) with the backend's weight cache."""

    def __init__(self, device=0):
        h = C.c_void_p()
        check(lib().ihip_create(device, C.byref(h)), "create")
        self.h = h
        self._keep = []

    def close(self):
        if self.h:
            lib().ihip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def info(self):
        name = C.create_string_buffer(256)
        mem, cus = C.c_uint64(), C.c_int()
        check(lib().ihip_device_info(self.h, name, 256, C.byref(mem), C.byref(cus)), "info")
        return name.value.decode(), mem.value, cus.value

    def alloc(self, nbytes):
        return Buffer(self, nbytes)

    def array(self, a):
        a = np.ascontiguousarray(a)
        b = Buffer(self, max(a.nbytes, 4))
        b.upload(a)
        return b

    def sync(self):
        check(lib().ihip_synchronize(self.h), "synchronize")

    def weight(self, host, dtype, out, cols, count=1):
        self._keep.append(host)
        d = C.c_uint64()
        check(lib().ihip_weight(self.h, _p(host), dtype, out, cols, count, C.byref(d)), "weight")
        return d.value

    def weight_f32(self, host):
        host = np.ascontiguousarray(host, np.float32)
        self._keep.append(host)
        d = C.c_uint64()
        check(lib().ihip_weight_f32(self.h, _p(host), host.size, C.byref(d)), "weight_f32")
        return d.value

    def linear(self, x, w, dtype, out, bias=None, mode=MODE_F32):
        x = np.ascontiguousarray(x, np.float32)
        rows, cols = x.shape
        y = np.empty((rows, out), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        if b is not None:
            self._keep.append(b)
        self._keep.append(w)
        check(lib().ihip_linear(self.h, _p(x), rows, cols, _p(w), dtype, out, _p(b), _p(y), mode),
              "linear")
        return y

    def record(self, i):
        check(lib().ihip_event_record(self.h, i), "event")

    def elapsed(self, a, b):
        ms = C.c_float()
        check(lib().ihip_event_elapsed(self.h, a, b, C.byref(ms)), "elapsed")
        return ms.value


# ---------------------------------------------------------------- models
class Tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int32), ("reserved", C.c_int32)]


_LAYER_TENSORS = ["input_norm", "q", "k", "v", "o", "q_bias", "k_bias", "v_bias", "o_bias",
                  "q_norm", "k_norm", "sinks", "post_norm", "gate", "up", "down", "router",
                  "router_bias", "exp_gate", "exp_up", "exp_down", "exp_gate_bias",
                  "exp_up_bias", "exp_down_bias"]


class LayerDesc(C.Structure):
    _fields_ = [(n, Tensor) for n in _LAYER_TENSORS] + [("window", C.c_int32), ("moe", C.c_int32)]


class ModelDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab", "hidden", "layers", "heads", "kv_heads",
                                          "head_dim", "ffn", "experts", "experts_used",
                                          "expert_ffn", "norm_topk", "max_positions")] + \
        [("rms_eps", C.c_float), ("swiglu_alpha", C.c_float), ("swiglu_limit", C.c_float),
         ("reserved0", C.c_float), ("rope_theta", C.c_double), ("rope_factor", C.c_double),
         ("rope_beta_fast", C.c_double), ("rope_beta_slow", C.c_double),
         ("rope_original", C.c_int32), ("rope_truncate", C.c_int32),
         ("rope_attention", C.c_double), ("embed", Tensor), ("final_norm", Tensor),
         ("head", Tensor), ("layer", C.POINTER(LayerDesc))]


class Model:
    """The decoder on the device (TQwen3Hip over TDecoderDevice)."""

    def __init__(self, ctx, spec, mode=MODE_Q8, kv_f16=False, max_tokens=1024):
        self.ctx = ctx
        self.spec = spec  # keeps the host tensors alive
        self.vocab = spec.vocab
        h = C.c_void_p()
        check(lib().ihip_model_create(ctx.h, C.addressof(spec.struct), mode, int(kv_f16),
                                      max_tokens, C.byref(h)), "model_create")
        self.h = h

    def close(self):
        if self.h:
            lib().ihip_model_destroy(self.h)
            self.h = None

    def __del__(self):
        if getattr(self, "h", None) and getattr(self.ctx, "h", None):
            self.close()

    def reset(self):
        check(lib().ihip_model_reset(self.h), "reset")

    def forward(self, ids, all_logits=False):
        ids = np.ascontiguousarray(ids, np.int32)
        lg = np.empty((len(ids) if all_logits else 1, self.vocab), np.float32)
        check(lib().ihip_model_forward(self.h, _p(ids), len(ids), _p(lg), int(all_logits)),
              "forward")
        return lg if all_logits else lg[0]

    def greedy(self, prompt, max_new):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max_new, np.int32)
        check(lib().ihip_model_greedy(self.h, _p(p), len(p), max_new, _p(out)), "greedy")
        return out

    def chunk(self, rows):
        check(lib().ihip_model_chunk(self.h, int(rows)), "chunk")

    def use_graphs(self, on):
        check(lib().ihip_model_use_graphs(self.h, int(on)), "use_graphs")

    def decode(self, first, steps):
        out = np.empty(steps, np.int32)
        check(lib().ihip_model_decode(self.h, int(first), steps, _p(out)), "decode")
        return out

    def timing(self):
        a, b = C.c_double(), C.c_double()
        check(lib().ihip_model_timing(self.h, C.byref(a), C.byref(b)), "timing")
        return a.value, b.value
