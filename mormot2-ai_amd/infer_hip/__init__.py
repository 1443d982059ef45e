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
LIB_PATH = os.environ.get("IHIP_LIB") or os.path.join(os.path.dirname(HERE), "libmormot_ai_hip.so")
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


class FormatError(HipError):
    """A damaged, hostile or unsupported file (IHIP_E_FORMAT, EInferError)."""


IHIP_E_ARG, IHIP_E_NOMEM, IHIP_E_FORMAT = -1, -6, -7


class Sampling(C.Structure):
    """TInferSampling (sampler.pas:46-59)."""
    _fields_ = [("temperature", C.c_double), ("top_k", C.c_int32), ("reserved", C.c_int32),
                ("top_p", C.c_double), ("min_p", C.c_double), ("seed", C.c_int64)]


def sampling(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, seed=0):
    return Sampling(temperature, top_k, 0, top_p, min_p, seed)


class GgufValue(C.Structure):
    _fields_ = [("key", C.c_char_p), ("vtype", C.c_int32), ("etype", C.c_int32),
                ("count", C.c_int64), ("data", C.c_void_p)]


class GgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
                ("shape", C.c_int64 * 4), ("count", C.c_int64), ("bytes", C.c_int64),
                ("data", C.c_void_p)]


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
            "ihip_kernel_timer": (i32, [vp, C.c_char_p, i64]),
            "ihip_kernel_timer_read": (i32, [vp, C.POINTER(i64), C.POINTER(C.c_double)]),
            "ihip_kernel_timer_report": (i32, [vp, C.c_char_p, i64]),
            "ihip_trace_buffer": (i32, [vp, u64, u64, i64, C.c_char_p]),
            "ihip_type_bytes": (u64, [i32, u64]),
            "ihip_weight": (i32, [vp, vp, i32, i64, i64, i64, C.POINTER(u64)]),
            "ihip_repack": (i32, [vp, vp, i32, i64, i64, i64, i32]),
            "ihip_weight_f32": (i32, [vp, vp, i64, C.POINTER(u64)]),
            "ihip_forget_weights": (i32, [vp, vp, vp]),
            "ihip_clear_weights": (i32, [vp]),
            "ihip_gpu_linear": (i32, [i32, i64]),
            "ihip_enqueue_linear_at": (i32, [vp, u64, i64, i64, i32, u64, i64, u64, u64, i32]),
            "ihip_enqueue_linear_at_static": (i32, [vp, u64, i64, i64, i32, u64, i64, u64, u64,
                                                    i32]),
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
            "ihip_enqueue_route": (i32, [vp, u64, i64, i64, i32, u64, u64, u64]),
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
            "ihip_model_check_route": (i32, [vp, i32]),
            "ihip_model_route_stats": (i32, [vp, vp, vp, vp]),
            "ihip_model_route_tape": (i32, [vp, vp, vp, i64]),
            "ihip_model_route_tape_stats": (i32, [vp, vp, vp, vp, vp]),
            "ihip_model_chunk": (i32, [vp, i64]),
            "ihip_enqueue_stream_read": (i32, [vp, u64, u64, u64]),
            "ihip_model_rotary": (i32, [vp, i64, i64, vp]),
            "ihip_model_new_context": (i32, [vp, C.POINTER(vp)]),
            "ihip_context_destroy": (None, [vp]),
            "ihip_model_context": (vp, [vp]),
            "ihip_context_forward": (i32, [vp, vp, i64, vp, i32]),
            "ihip_context_forward_embeds": (i32, [vp, vp, i64, vp, i32, vp, i32]),
            "ihip_context_reuse": (i32, [vp, vp, i64, C.POINTER(i64)]),
            "ihip_context_truncate": (i32, [vp, i64]),
            "ihip_context_length": (i32, [vp, C.POINTER(i64), C.POINTER(i64)]),
            "ihip_context_set_checkpoints": (i32, [vp, i32, i64]),
            "ihip_context_checkpoints": (i32, [vp, vp, i64, C.POINTER(i64)]),
            "ihip_context_greedy": (i32, [vp, vp, i64, i64, vp]),
            "ihip_context_decode": (i32, [vp, C.c_int32, i64, vp]),
            "ihip_native_decode": (i32, [vp, vp, i64, i64, C.POINTER(Sampling), i64, vp, i64, i64,
                                         vp, C.POINTER(i64), C.POINTER(i64), C.POINTER(C.c_int)]),
            "ihip_prompt_cache_create": (i32, [vp, i64, C.POINTER(vp)]),
            "ihip_prompt_cache_destroy": (None, [vp]),
            "ihip_prompt_cache_set_slots": (i32, [vp, i64]),
            "ihip_prompt_cache_clear": (i32, [vp]),
            "ihip_prompt_cache_acquire": (i32, [vp, vp, i64, C.POINTER(vp)]),
            "ihip_prompt_cache_release": (i32, [vp, vp, i64]),
            "ihip_prompt_cache_stats": (i32, [vp, C.POINTER(i64), C.POINTER(i64), C.POINTER(i64),
                                              C.POINTER(i64)]),
            "ihip_model_timing": (i32, [vp, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
            "ihip_synth_blocks": (i32, [vp, i32, i64, i64, u64, i32, i32, i32]),
            "ihip_synth_normal": (i32, [vp, i32, i64, i64, u64, C.c_float, i32]),
            "ihip_gguf_open": (i32, [C.c_char_p, C.POINTER(vp)]),
            "ihip_gguf_open_mem": (i32, [vp, i64, C.POINTER(vp)]),
            "ihip_gguf_close": (None, [vp]),
            "ihip_gguf_alignment": (i64, [vp]),
            "ihip_gguf_value_count": (i64, [vp]),
            "ihip_gguf_tensor_count": (i64, [vp]),
            "ihip_gguf_value_at": (i32, [vp, i64, C.POINTER(GgufValue)]),
            "ihip_gguf_find": (i64, [vp, C.c_char_p]),
            "ihip_gguf_str": (i32, [vp, C.c_char_p, C.POINTER(vp), C.POINTER(i64)]),
            "ihip_gguf_int": (i32, [vp, C.c_char_p, C.POINTER(i64)]),
            "ihip_gguf_float": (i32, [vp, C.c_char_p, C.POINTER(C.c_double)]),
            "ihip_gguf_bool": (i32, [vp, C.c_char_p, C.POINTER(i32)]),
            "ihip_gguf_bool_def": (i32, [vp, C.c_char_p, i32, C.POINTER(i32)]),
            "ihip_gguf_array": (i32, [vp, C.c_char_p, i32, i64, C.POINTER(vp), C.POINTER(i64)]),
            "ihip_gguf_strings": (i32, [vp, C.c_char_p, i64, i64, C.POINTER(vp),
                                        C.POINTER(i64)]),
            "ihip_gguf_tensor_at": (i32, [vp, i64, C.POINTER(GgufTensor)]),
            "ihip_gguf_find_tensor": (i64, [vp, C.c_char_p]),
            "ihip_gguf_weight": (i32, [vp, C.c_char_p, i32, i32, C.POINTER(i64), C.POINTER(vp)]),
            "ihip_gguf_model_desc": (i32, [vp, C.POINTER(vp)]),
            "ihip_sampler_create": (i32, [vp, C.POINTER(Sampling), i64, C.POINTER(vp)]),
            "ihip_sampler_destroy": (None, [vp]),
            "ihip_enqueue_sample": (i32, [vp, vp, u64, i64, u64]),
            "ihip_model_sampling": (i32, [vp, C.POINTER(Sampling)]),
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
        raise (FormatError if rc == IHIP_E_FORMAT else HipError)(f"{what}: status {rc}: {msg}")


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

    def kernel_timer(self, prefix, capacity=4096):
        """Time every later direct launch of kernels named prefix* by their
        own dispatch (None: stop)."""
        check(lib().ihip_kernel_timer(self.h, prefix.encode() if prefix else None, capacity),
              "kernel_timer")

    def kernel_timer_read(self):
        """(launches, total ms) since the last read."""
        n, ms = C.c_int64(), C.c_double()
        check(lib().ihip_kernel_timer_read(self.h, C.byref(n), C.byref(ms)), "kernel_timer_read")
        return n.value, ms.value

    def kernel_timer_report(self):
        """{kernel: (launches, total ms)} since the last read."""
        buf = C.create_string_buffer(1 << 16)
        check(lib().ihip_kernel_timer_report(self.h, buf, len(buf)), "kernel_timer_report")
        out = {}
        for line in buf.value.decode().splitlines():
            name, n, ms = line.split()
            out[name] = (int(n), float(ms))
        return out

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
_LIN_TENSORS = ["lin_qkv", "lin_z", "lin_b", "lin_a", "lin_out", "lin_conv", "lin_dt_bias",
                "lin_neg_a", "lin_norm"]
MIXER_ATTENTION, MIXER_DELTANET = 0, 1
FFN_DENSE, FFN_MOE, FFN_DENSE_MOE = 0, 1, 2
ACT_SILU, ACT_GELU_TANH = 0, 1
_GEMMA_TENSORS = ["attn_out_norm", "ffn_out_norm", "dense_out_norm", "moe_in_norm", "moe_out_norm",
                  "router_norm", "expert_scale", "scalar"]


class LayerDesc(C.Structure):
    _fields_ = [(n, Tensor) for n in _LAYER_TENSORS] + [
        ("window", C.c_int32), ("moe", C.c_int32), ("mixer", C.c_int32),
        ("output_gate", C.c_int32)] + [(n, Tensor) for n in _LIN_TENSORS] + [
        (n, C.c_int32) for n in ("head_dim", "kv_heads", "k_is_v", "rope_set", "exp_gate_up",
                                 "no_rope")] + [(n, Tensor) for n in _GEMMA_TENSORS]


class ModelDesc(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab", "hidden", "layers", "heads", "kv_heads",
                                          "head_dim", "ffn", "experts", "experts_used",
                                          "expert_ffn", "norm_topk", "max_positions")] + \
        [("rms_eps", C.c_float), ("swiglu_alpha", C.c_float), ("swiglu_limit", C.c_float),
         ("reserved0", C.c_float), ("rope_theta", C.c_double), ("rope_factor", C.c_double),
         ("rope_beta_fast", C.c_double), ("rope_beta_slow", C.c_double),
         ("rope_original", C.c_int32), ("rope_truncate", C.c_int32),
         ("rope_attention", C.c_double), ("embed", Tensor), ("final_norm", Tensor),
         ("head", Tensor), ("layer", C.POINTER(LayerDesc))] + \
        [(n, C.c_int32) for n in ("rope_dims", "lin_key_heads", "lin_value_heads",
                                  "lin_key_dim", "lin_value_dim", "lin_conv", "lin_tiled",
                                  "activation", "value_norm")] + \
        [("embed_scale", C.c_float), ("reserved2", C.c_float), ("attention_scale", C.c_double),
         ("logit_softcap", C.c_double), ("rope2_theta", C.c_double), ("rope2_pairs", C.c_int32),
         ("reserved3", C.c_int32)]


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

    def sampling(self, **kw):
        """Draw the next tokens with these settings (None: the argmax)."""
        s = sampling(**kw) if kw else None
        check(lib().ihip_model_sampling(self.h, C.byref(s) if s is not None else None), "sampling")

    def decode(self, first, steps):
        out = np.empty(steps, np.int32)
        check(lib().ihip_model_decode(self.h, int(first), steps, _p(out)), "decode")
        return out

    def check_route(self, on):
        """CheckRoute: compare every one-row device route with the host's
        TDecoderModel.Route (decode without graphs meanwhile)."""
        check(lib().ihip_model_check_route(self.h, int(on)), "check_route")

    def route_stats(self):
        """(RouteChecks, RouteMismatches, RouteMaxDiff)."""
        a, b, d = C.c_int64(), C.c_int64(), C.c_double()
        check(lib().ihip_model_route_stats(self.h, C.byref(a), C.byref(b), C.byref(d)), "route_stats")
        return a.value, b.value, d.value

    def route_tape(self, ids=None, weights=None):
        """TDecoderRouteTape replay: the rows routed from now on take these
        picks and weights [rows, experts_used] in turn (None: off)."""
        if ids is None:
            check(lib().ihip_model_route_tape(self.h, None, None, 0), "route_tape")
            return
        self._tape = (np.ascontiguousarray(ids, np.int32), np.ascontiguousarray(weights, np.float32))
        check(lib().ihip_model_route_tape(self.h, _p(self._tape[0]), _p(self._tape[1]),
                                          self._tape[0].shape[0]), "route_tape")

    def route_tape_stats(self):
        """(routes replayed, rows the device chose otherwise, the largest
        router gap of those, rows pending)."""
        a, b, p = C.c_int64(), C.c_int64(), C.c_int64()
        g = C.c_double()
        check(lib().ihip_model_route_tape_stats(self.h, C.byref(a), C.byref(b), C.byref(g),
                                                C.byref(p)), "route_tape_stats")
        return a.value, b.value, g.value, p.value

    def timing(self):
        a, b = C.c_double(), C.c_double()
        check(lib().ihip_model_timing(self.h, C.byref(a), C.byref(b)), "timing")
        return a.value, b.value

    def new_context(self):
        """A new, empty context of this model (NewDeviceContext)."""
        return ModelContext(self)

    def context(self):
        """The model's own context (the one forward/greedy/decode use)."""
        return ModelContext(self, own=True)


class ModelContext:
    """One sequence on the device (a TDecoderContext of TDecoderDevice): its
    KV cache, grown as tokens come; the weights are the model's."""

    def __init__(self, model, own=False):
        self.model = model
        self.own = own
        self.vocab = model.vocab
        self.hidden = model.spec.struct.hidden
        if own:
            self.h = C.c_void_p(lib().ihip_model_context(model.h))
        else:
            h = C.c_void_p()
            check(lib().ihip_model_new_context(model.h, C.byref(h)), "new_context")
            self.h = h

    def close(self):
        # a context of a model whose device context is gone is gone with it
        if self.h and not self.own and self.model.h and getattr(self.model.ctx, "h", None):
            lib().ihip_context_destroy(self.h)
        self.h = None

    def __del__(self):
        if getattr(self, "h", None) and getattr(self.model, "h", None):
            self.close()

    def forward(self, ids, all_logits=False):
        ids = np.ascontiguousarray(ids, np.int32)
        lg = np.empty((len(ids) if all_logits else 1, self.vocab), np.float32)
        check(lib().ihip_context_forward(self.h, _p(ids), len(ids), _p(lg), int(all_logits)),
              "forward")
        return lg if all_logits else lg[0]

    def forward_embeds(self, embeds, all_logits=False, normed=False, logits=True, head=0):
        """ForwardEmbeds: rows [count, hidden] in place of token embeddings;
        returns (logits or None, the last row's final norm or None)."""
        e = np.ascontiguousarray(embeds, np.float32).reshape(-1, self.hidden)
        n = e.shape[0]
        lg = np.empty((n if all_logits else 1, self.vocab), np.float32) if logits else None
        nv = np.empty(self.hidden, np.float32) if normed else None
        check(lib().ihip_context_forward_embeds(self.h, _p(e), n, _p(lg), int(all_logits), _p(nv),
                                                head), "forward_embeds")
        if lg is not None and not all_logits:
            lg = lg[0]
        return lg, nv

    def reuse(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        kept = C.c_int64()
        check(lib().ihip_context_reuse(self.h, _p(ids), len(ids), C.byref(kept)), "reuse")
        return kept.value

    def truncate(self, length):
        check(lib().ihip_context_truncate(self.h, int(length)), "truncate")

    def length(self):
        n, cap = C.c_int64(), C.c_int64()
        check(lib().ihip_context_length(self.h, C.byref(n), C.byref(cap)), "length")
        return n.value, cap.value

    def set_checkpoints(self, token_id, max_count=4):
        """CheckpointId / MaxCheckpoints: restore points of the recurrent
        state before every token_id of an aligned forward (-1: none)."""
        check(lib().ihip_context_set_checkpoints(self.h, int(token_id), int(max_count)),
              "set_checkpoints")

    def checkpoints(self):
        """The lengths of the restore points held, the oldest first."""
        out = np.zeros(64, np.int64)
        n = C.c_int64()
        check(lib().ihip_context_checkpoints(self.h, _p(out), len(out), C.byref(n)), "checkpoints")
        return out[:min(n.value, len(out))].tolist()

    def greedy(self, prompt, max_new):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max_new, np.int32)
        check(lib().ihip_context_greedy(self.h, _p(p), len(p), max_new, _p(out)), "greedy")
        return out

    def decode(self, first, steps):
        out = np.empty(steps, np.int32)
        check(lib().ihip_context_decode(self.h, int(first), steps, _p(out)), "decode")
        return out

    def native_decode(self, prompt, max_new, sampling_kw=None, stop=(), max_context=0,
                      draw_ids=0):
        """NativeDecode (llm.native.pas:2135-2185) on this context: returns
        (tokens, prompt tokens reused from the cache, stopped by a stop id).
        sampling_kw: the TInferSampling settings (None: greedy)."""
        p = np.ascontiguousarray(prompt, np.int32)
        st = np.ascontiguousarray(list(stop), np.int32)
        out = np.empty(max(int(max_new), 1), np.int32)
        n, reused, stopped = C.c_int64(), C.c_int64(), C.c_int()
        smp = sampling(**sampling_kw) if sampling_kw else None
        check(lib().ihip_native_decode(self.h, _p(p), len(p), int(max_new),
                                       C.byref(smp) if smp is not None else None, int(draw_ids),
                                       _p(st) if len(st) else None, len(st), int(max_context),
                                       _p(out), C.byref(n), C.byref(reused), C.byref(stopped)),
              "native_decode")
        return out[:n.value].copy(), reused.value, bool(stopped.value)


class PromptCache:
    """TNativePromptCache (llm.native.pas:2192-2350): idle contexts of a model
    kept between requests; acquire() hands out the one sharing the longest
    start with a prompt, release() takes it back."""

    def __init__(self, model, slots=1):
        self.model = model
        h = C.c_void_p()
        check(lib().ihip_prompt_cache_create(model.h, int(slots), C.byref(h)), "prompt_cache")
        self.h = h

    def close(self):
        if self.h and self.model.h and getattr(self.model.ctx, "h", None):
            lib().ihip_prompt_cache_destroy(self.h)
        self.h = None

    def __del__(self):
        if getattr(self, "h", None) and getattr(self.model, "h", None):
            self.close()

    def set_slots(self, slots):
        check(lib().ihip_prompt_cache_set_slots(self.h, int(slots)), "set_slots")

    def clear(self):
        check(lib().ihip_prompt_cache_clear(self.h), "clear")

    def acquire(self, prompt):
        """A context for the prompt, the caller's until released."""
        p = np.ascontiguousarray(prompt, np.int32)
        h = C.c_void_p()
        check(lib().ihip_prompt_cache_acquire(self.h, _p(p), len(p), C.byref(h)), "acquire")
        ctx = ModelContext.__new__(ModelContext)
        ctx.model, ctx.own, ctx.vocab = self.model, False, self.model.vocab
        ctx.hidden = self.model.spec.struct.hidden
        ctx.h = h
        return ctx

    def release(self, ctx, reused):
        check(lib().ihip_prompt_cache_release(self.h, ctx.h, int(reused)), "release")
        ctx.h = None  # the cache's again

    def stats(self):
        r, hi, ru, idle = C.c_int64(), C.c_int64(), C.c_int64(), C.c_int64()
        check(lib().ihip_prompt_cache_stats(self.h, C.byref(r), C.byref(hi), C.byref(ru),
                                            C.byref(idle)), "stats")
        return {"requests": r.value, "hits": hi.value, "reused": ru.value, "idle": idle.value}


def native_generate(cache, prompt, max_new, sampling_kw=None, stop=(), max_context=0, draw_ids=0):
    """TNativeLlmClient.Generate's device part (llm.native.pas:2447-2481): a
    context from the prompt cache, NativeDecode on it, the context back to
    the cache (freed instead when the request fails)."""
    ctx = cache.acquire(prompt)
    try:
        out = ctx.native_decode(prompt, max_new, sampling_kw, stop, max_context, draw_ids)
    except Exception:
        ctx.close()
        raise
    cache.release(ctx, out[1])
    return out


# ---------------------------------------------------------------- GGUF
GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, \
    GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64 = range(13)


class Gguf:
    """A validated, memory-mapped GGUF v3 file (TGgufFile,
    src/infer/mormot.ai.infer.loader.gguf.pas:94-170): path, or content=bytes
    for CreateFromContent. A defect raises FormatError."""

    def __init__(self, path=None, content=None):
        h = C.c_void_p()
        if content is not None:
            buf = C.create_string_buffer(bytes(content), len(content))
            rc = lib().ihip_gguf_open_mem(buf, len(content), C.byref(h))
        else:
            rc = lib().ihip_gguf_open(os.fsencode(path), C.byref(h))
        check(rc, "gguf")
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().ihip_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def alignment(self):
        return lib().ihip_gguf_alignment(self.h)

    def keys(self):
        out = []
        v = GgufValue()
        for i in range(lib().ihip_gguf_value_count(self.h)):
            check(lib().ihip_gguf_value_at(self.h, i, C.byref(v)), "value_at")
            out.append(v.key.decode())
        return out

    def has(self, key):
        return lib().ihip_gguf_find(self.h, key.encode()) >= 0

    def str(self, key):
        p, n = C.c_void_p(), C.c_int64()
        check(lib().ihip_gguf_str(self.h, key.encode(), C.byref(p), C.byref(n)), "str")
        return C.string_at(p, n.value).decode()

    def int(self, key):
        v = C.c_int64()
        check(lib().ihip_gguf_int(self.h, key.encode(), C.byref(v)), "int")
        return v.value

    def float(self, key):
        v = C.c_double()
        check(lib().ihip_gguf_float(self.h, key.encode(), C.byref(v)), "float")
        return v.value

    def bool(self, key, default=None):
        v = C.c_int()
        if default is None:
            check(lib().ihip_gguf_bool(self.h, key.encode(), C.byref(v)), "bool")
        else:
            check(lib().ihip_gguf_bool_def(self.h, key.encode(), int(default), C.byref(v)), "bool")
        return bool(v.value)

    def array(self, key, elem, count=-1):
        """A fixed-size element array as numpy (a copy)."""
        dt = {GGUF_UINT8: np.uint8, GGUF_INT8: np.int8, GGUF_UINT16: np.uint16,
              GGUF_INT16: np.int16, GGUF_UINT32: np.uint32, GGUF_INT32: np.int32,
              GGUF_FLOAT32: np.float32, GGUF_BOOL: np.uint8, GGUF_UINT64: np.uint64,
              GGUF_INT64: np.int64, GGUF_FLOAT64: np.float64}[elem]
        p, n = C.c_void_p(), C.c_int64()
        check(lib().ihip_gguf_array(self.h, key.encode(), elem, count, C.byref(p), C.byref(n)),
              "array")
        return np.frombuffer(C.string_at(p, n.value * np.dtype(dt).itemsize), dt).copy()

    def strings(self, key):
        v = GgufValue()
        i = lib().ihip_gguf_find(self.h, key.encode())
        n = 0
        if i >= 0:
            check(lib().ihip_gguf_value_at(self.h, i, C.byref(v)), "value_at")
            n = v.count if v.vtype == GGUF_ARRAY else 0
        ptrs, lens = (C.c_void_p * max(n, 1))(), (C.c_int64 * max(n, 1))()
        check(lib().ihip_gguf_strings(self.h, key.encode(), 0, n, ptrs, lens), "strings")
        return [C.string_at(ptrs[j], lens[j]).decode(errors="surrogateescape") for j in range(n)]

    def tensors(self):
        out = []
        t = GgufTensor()
        for i in range(lib().ihip_gguf_tensor_count(self.h)):
            check(lib().ihip_gguf_tensor_at(self.h, i, C.byref(t)), "tensor_at")
            out.append(dict(name=t.name.decode(), dtype=t.dtype, shape=tuple(t.shape[:t.ndim]),
                            count=t.count, bytes=t.bytes, data=t.data))
        return out

    def tensor(self, name):
        """The tensor named name, or None (FindTensor)."""
        i = lib().ihip_gguf_find_tensor(self.h, name.encode())
        if i < 0:
            return None
        t = GgufTensor()
        check(lib().ihip_gguf_tensor_at(self.h, i, C.byref(t)), "tensor_at")
        return dict(name=name, dtype=t.dtype, shape=tuple(t.shape[:t.ndim]), count=t.count,
                    bytes=t.bytes, data=t.data)

    def weight(self, name, dtype, dims):
        d = (C.c_int64 * len(dims))(*dims)
        p = C.c_void_p()
        check(lib().ihip_gguf_weight(self.h, name.encode(), dtype, len(dims), d, C.byref(p)),
              "weight")
        return p.value


class GgufSpec:
    """The decoder of a qwen3 / qwen3moe / gpt-oss GGUF file as a model
    description (NewDecoderModelFromGguf, decoder.pas:3491-3510): pass it to
    Model (the device) or to the CPU oracle like a synthetic Spec."""

    def __init__(self, path=None, content=None):
        self.file = Gguf(path, content)
        p = C.c_void_p()
        check(lib().ihip_gguf_model_desc(self.file.h, C.byref(p)), "gguf model")
        self.struct = ModelDesc.from_address(p.value)
        self.vocab = self.struct.vocab
        self.layers = [self.struct.layer[i] for i in range(self.struct.layers)]
        d = self.struct
        self.cfg = dict(vocab=d.vocab, hidden=d.hidden, layers=d.layers, heads=d.heads,
                        kv_heads=d.kv_heads, head_dim=d.head_dim, ffn=d.ffn, experts=d.experts,
                        experts_used=d.experts_used, expert_ffn=d.expert_ffn)

    def close(self):
        self.file.close()


class Sampler:
    """TInferSampler on the device (ihip_sampler): draws with its own
    splitmix64 stream, kept on the device."""

    def __init__(self, ctx, n_max, **kw):
        self.ctx = ctx
        h = C.c_void_p()
        s = sampling(**kw)
        check(lib().ihip_sampler_create(ctx.h, C.byref(s), n_max, C.byref(h)), "sampler")
        self.h = h

    def enqueue(self, logits_ptr, n, out_ptr):
        check(lib().ihip_enqueue_sample(self.ctx.h, self.h, logits_ptr, n, out_ptr), "sample")

    def close(self):
        if getattr(self, "h", None) and getattr(self.ctx, "h", None):
            lib().ihip_sampler_destroy(self.h)
        self.h = None

    def __del__(self):
        self.close()
