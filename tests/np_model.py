"""An independent float64 numpy forward of the decoder families (test
infrastructure): the oracle's decoder composition (oracle/model.c) is pinned
against it in its F32 arithmetic. It follows the published architectures as
decoder.pas implements them - pre-norm attention with per-head q/k norms,
rotate_half RoPE, causal GQA with window and sinks, pre-norm dense SwiGLU or
routed experts (softmax top-k, renormalised), final norm and head - written
from the formulas, not from the oracle's C."""
import ctypes as C

import numpy as np

import oracle_lib as O


def _w(t, rows, cols, offset=0):
    """Dequantized [rows, cols] from an ihip_tensor (float64)."""
    nb = O.row_bytes(t.dtype, cols) * rows
    raw = np.ctypeslib.as_array(C.cast(int(t.data) + int(offset), C.POINTER(C.c_uint8)), (nb,))
    return O.dequant(np.ascontiguousarray(raw), t.dtype, rows, cols).astype(np.float64)


def _v(t, n):
    if not t.data:
        return None
    return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), (n,)).astype(np.float64)


def _rms(x, w, eps):
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * w


class NumpyModel:
    def __init__(self, spec):
        self.s = spec
        d = spec.struct
        self.d = d
        self.keys = [[] for _ in range(d.layers)]
        self.vals = [[] for _ in range(d.layers)]
        self.length = 0

    def forward(self, ids):
        d, s = self.d, self.s
        H, hd, nh, nk = d.hidden, d.head_dim, d.heads, d.kv_heads
        n = len(ids)
        emb = d.embed
        x = np.stack([_w(emb, d.vocab, H)[i] for i in ids]) if d.vocab * H < 50_000_000 else None
        half = hd // 2
        cs = np.empty(n * hd, np.float32)
        O.lib().orc_rotary(C.addressof(d), self.length, n, cs.ctypes.data)
        cos = cs[:n * half].reshape(n, half).astype(np.float64)
        sin = cs[n * half:].reshape(n, half).astype(np.float64)

        def rope(t, heads):
            t = t.reshape(n, heads, hd)
            a, b = t[..., :half], t[..., half:]
            c, sn = cos[:, None, :], sin[:, None, :]
            return np.concatenate([a * c - b * sn, b * c + a * sn], axis=-1).reshape(n, heads * hd)

        for li in range(d.layers):
            L = s.layers[li]
            h = _rms(x, _v(L.input_norm, H), d.rms_eps)

            def lin(inp, t, rows, cols, bias):
                y = inp @ _w(t, rows, cols).T
                return y + bias if bias is not None else y

            q = lin(h, L.q, nh * hd, H, _v(L.q_bias, nh * hd))
            k = lin(h, L.k, nk * hd, H, _v(L.k_bias, nk * hd))
            v = lin(h, L.v, nk * hd, H, _v(L.v_bias, nk * hd))
            if L.q_norm.data:
                q = _rms(q.reshape(n, nh, hd), _v(L.q_norm, hd), d.rms_eps).reshape(n, -1)
                k = _rms(k.reshape(n, nk, hd), _v(L.k_norm, hd), d.rms_eps).reshape(n, -1)
            q, k = rope(q, nh), rope(k, nk)
            self.keys[li].extend(list(k))
            self.vals[li].extend(list(v))
            K = np.array(self.keys[li]).reshape(-1, nk, hd)
            V = np.array(self.vals[li]).reshape(-1, nk, hd)
            sinks = _v(L.sinks, nh)
            att = np.zeros((n, nh * hd))
            for r in range(n):
                total = self.length + r + 1
                first = max(0, total - L.window) if L.window > 0 else 0
                for hh in range(nh):
                    g = hh // (nh // nk)
                    sc = K[first:total, g] @ q[r, hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                    m = sc.max() if sinks is None else max(sc.max(), sinks[hh])
                    e = np.exp(sc - m)
                    den = e.sum() + (np.exp(sinks[hh] - m) if sinks is not None else 0.0)
                    att[r, hh * hd:(hh + 1) * hd] = (e / den) @ V[first:total, g]
            x = x + lin(att, L.o, H, nh * hd, _v(L.o_bias, H))
            h = _rms(x, _v(L.post_norm, H), d.rms_eps)
            alpha, limit = d.swiglu_alpha, d.swiglu_limit

            def act(g, u):
                if limit > 0:
                    g = np.minimum(g, limit)
                    u = np.clip(u, -limit, limit)
                    return (u + 1) * g / (1 + np.exp(-alpha * g))
                return g / (1 + np.exp(-g)) * u

            if not L.moe:
                F = d.ffn
                y = lin(act(lin(h, L.gate, F, H, None), lin(h, L.up, F, H, None)), L.down, H, F, None)
            else:
                E, Kt, FI = d.experts, d.experts_used, d.expert_ffn
                lg = lin(h, L.router, E, H, _v(L.router_bias, E))
                y = np.zeros_like(x)
                gb = O.row_bytes(L.exp_gate.dtype, H) * FI
                db = O.row_bytes(L.exp_down.dtype, FI) * H
                egb, eub, edb = (_v(L.exp_gate_bias, E * FI), _v(L.exp_up_bias, E * FI),
                                 _v(L.exp_down_bias, E * H))
                for r in range(n):
                    p = np.exp(lg[r] - lg[r].max())
                    p /= p.sum()
                    top = np.argsort(-lg[r], kind="stable")[:Kt]
                    w = p[top] / p[top].sum() if d.norm_topk else p[top]
                    for e, we in sorted(zip(top, w)):
                        ge = h[r] @ _w(L.exp_gate, FI, H, e * gb).T
                        ue = h[r] @ _w(L.exp_up, FI, H, e * gb).T
                        if egb is not None:
                            ge = ge + egb[e * FI:(e + 1) * FI]
                            ue = ue + eub[e * FI:(e + 1) * FI]
                        de = act(ge, ue) @ _w(L.exp_down, H, FI, e * db).T
                        if edb is not None:
                            de = de + edb[e * H:(e + 1) * H]
                        y[r] += we * de
            x = x + y
        self.length += n
        h = _rms(x, _v(d.final_norm, H), d.rms_eps)
        head = d.head if d.head.data else d.embed
        return h @ _w(head, d.vocab, H).T
