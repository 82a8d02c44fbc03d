"""ctypes wrapper of the C oracle (libgemma_oracle.so).

TEST INFRASTRUCTURE ONLY: the oracle the HIP path is tested against. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libgemma_oracle.so")

_F = ctypes.POINTER(ctypes.c_float)
_U8 = ctypes.POINTER(ctypes.c_uint8)
_U16 = ctypes.POINTER(ctypes.c_uint16)
_U32 = ctypes.POINTER(ctypes.c_uint32)
_I32 = ctypes.POINTER(ctypes.c_int32)
_P = ctypes.c_void_p

GOR_HIDDEN, GOR_NORMED, GOR_LOGITS, GOR_LAYER_HIDDEN, GOR_K_CACHE, GOR_V_CACHE, GOR_Q, GOR_ATTN_OUT = range(8)


class GorConfig(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int32), ("num_layers", ctypes.c_int32), ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("intermediate_size", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32), ("context_length", ctypes.c_int32), ("rms_norm_eps", ctypes.c_float),
        ("rope_theta_global", ctypes.c_float), ("rope_theta_local", ctypes.c_float),
        ("swa_period", ctypes.c_int32), ("sliding_window", ctypes.c_int32),
    ]


_SIGS = {
    "gor_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "gor_f16_to_f32_n": (None, [_U16, ctypes.c_size_t, _F]),
    "gor_q8_0_dequant": (None, [_U8, ctypes.c_size_t, _F]),
    "gor_q8_0_pack36": (None, [_U8, ctypes.c_size_t, _U32]),
    "gor_embed": (None, [_U8, ctypes.c_int, ctypes.c_int, _F]),
    "gor_rms_norm": (None, [_F, _F, _F, ctypes.c_int, ctypes.c_float]),
    "gor_fused_norm_add": (None, [_F, _F, _F, _F, ctypes.c_int, ctypes.c_float]),
    "gor_linear_q8": (None, [_U8, _F, _F, ctypes.c_int, ctypes.c_int]),
    "gor_gelu_mul": (None, [_F, _F, _F, ctypes.c_int]),
    "gor_rope_freq": (ctypes.c_float, [ctypes.c_int, ctypes.c_int, ctypes.c_float]),
    "gor_per_head_norm_rope": (None, [_F, _F, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                                      ctypes.c_float]),
    "gor_attention": (None, [_F, _F, _F, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                             ctypes.c_float, _F, _F]),
    "gor_argmax": (ctypes.c_int, [_F, ctypes.c_int]),
    "gor_topk256": (None, [_F, ctypes.c_int, _F, _U32]),
    "gor_sample_candidates": (ctypes.c_int, [_F, _U32, _U32, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                                             ctypes.c_double]),
    "gor_model_create": (_P, [ctypes.POINTER(GorConfig)]),
    "gor_model_set_tensor": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_uint32, _P, ctypes.c_size_t]),
    "gor_model_destroy": (None, [_P]),
    "gor_model_reset_kv": (None, [_P]),
    "gor_model_forward": (ctypes.c_int, [_P, ctypes.c_int, ctypes.c_int]),
    "gor_model_lm_head": (None, [_P]),
    "gor_model_select": (ctypes.c_int, [_P, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                                        _I32, ctypes.c_int]),
    "gor_model_buffer": (_F, [_P, ctypes.c_int, ctypes.c_int]),
    "gor_set_threads": (None, [ctypes.c_int]),
    "gor_get_threads": (ctypes.c_int, []),
}

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run oracle/build.py)")
        L = ctypes.CDLL(LIB_PATH)
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _LIB = L
    return _LIB


def _f(a):
    return a.ctypes.data_as(_F)


def _u8(a):
    return a.ctypes.data_as(_U8)


def _u32(a):
    return a.ctypes.data_as(_U32)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- kernel-level functions ----------------------------------------------

def f16_to_f32(codes: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint16)
    out = np.empty(c.size, np.float32)
    lib().gor_f16_to_f32_n(c.ctypes.data_as(_U16), c.size, _f(out))
    return out


def q8_0_dequant(blocks: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, np.float32)
    lib().gor_q8_0_dequant(_u8(b), n, _f(out))
    return out


def q8_0_pack36(blocks: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n // 32 * 9, np.uint32)
    lib().gor_q8_0_pack36(_u8(b), n, _u32(out))
    return out


def embed(emb_blocks: np.ndarray, token: int, hidden: int) -> np.ndarray:
    b = np.ascontiguousarray(emb_blocks, dtype=np.uint8)
    out = np.empty(hidden, np.float32)
    lib().gor_embed(_u8(b), token, hidden, _f(out))
    return out


def rms_norm(x, w, eps=1e-6):
    x, w = f32(x), f32(w)
    out = np.empty_like(x)
    lib().gor_rms_norm(_f(x), _f(w), _f(out), x.size, eps)
    return out


def fused_norm_add(x, w, res, eps=1e-6):
    x, w, res = f32(x), f32(w), f32(res)
    out = np.empty_like(x)
    lib().gor_fused_norm_add(_f(x), _f(w), _f(res), _f(out), x.size, eps)
    return out


def linear_q8(w_blocks: np.ndarray, x, rows: int) -> np.ndarray:
    b = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    x = f32(x)
    y = np.empty(rows, np.float32)
    lib().gor_linear_q8(_u8(b), _f(x), _f(y), rows, x.size)
    return y


def gelu_mul(g, u):
    g, u = f32(g), f32(u)
    out = np.empty_like(g)
    lib().gor_gelu_mul(_f(g), _f(u), _f(out), g.size)
    return out


def rope_freq(i, head_dim, theta):
    return lib().gor_rope_freq(i, head_dim, theta)


def per_head_norm_rope(data, w, n_heads, head_dim, eps, pos, theta):
    d = f32(data).copy()
    w = f32(w)
    lib().gor_per_head_norm_rope(_f(d), _f(w), n_heads, head_dim, eps, pos, theta)
    return d


def attention(q, k_cache, v_cache, n_q, n_kv, head_dim, t_lo, t_hi, scale):
    q, kc, vc = f32(q), f32(k_cache), f32(v_cache)
    seq = t_hi - t_lo + 1
    scores = np.empty(n_q * seq, np.float32)
    out = np.empty(n_q * head_dim, np.float32)
    lib().gor_attention(_f(q), _f(kc), _f(vc), n_q, n_kv, head_dim, t_lo, t_hi, scale, _f(scores), _f(out))
    return out, scores.reshape(n_q, seq)


def argmax(logits) -> int:
    x = f32(logits)
    return lib().gor_argmax(_f(x), x.size)


def topk256(logits):
    x = f32(logits)
    v = np.empty(256, np.float32)
    i = np.empty(256, np.uint32)
    lib().gor_topk256(_f(x), x.size, _f(v), _u32(i))
    return v, i


def seen_bitmap(ids):
    """Penalty set as the 8192-word bitmap gor_sample_candidates reads."""
    bm = np.zeros(8192, np.uint32)
    for t in ids:
        bm[t >> 5] |= np.uint32(1 << (t & 31))
    return bm


def sample_candidates(vals, ids, seen_ids, temperature, top_p, rep_penalty, u) -> int:
    v = f32(vals)
    i = np.ascontiguousarray(ids, dtype=np.uint32)
    bm = seen_bitmap(seen_ids) if len(seen_ids) else np.zeros(8192, np.uint32)
    return lib().gor_sample_candidates(_f(v), _u32(i), _u32(bm), temperature, top_p, rep_penalty, u)


def set_threads(n: int):
    lib().gor_set_threads(int(n))


def get_threads() -> int:
    return int(lib().gor_get_threads())


# ---- whole model ----------------------------------------------------------

class OracleModel:
    """The reference forward pass on the CPU. Q8_0 tensors are borrowed from
    the `tensors` dict (kept alive here); norm tensors are copied."""

    def __init__(self, shape, tensors: dict):
        self.shape = shape
        self._keep = tensors
        c = GorConfig(shape.hidden, shape.layers, shape.n_q, shape.n_kv, shape.head_dim, shape.inter, shape.vocab,
                      shape.ctx, shape.eps, shape.theta_global, shape.theta_local, shape.swa_period, shape.window)
        self.m = lib().gor_model_create(ctypes.byref(c))
        if not self.m:
            raise RuntimeError("gor_model_create failed")
        for name, (t, dims, data) in tensors.items():
            arr = np.ascontiguousarray(data)
            rc = lib().gor_model_set_tensor(self.m, name.encode(), t, arr.ctypes.data, arr.nbytes)
            if rc != 0:
                raise RuntimeError(f"oracle rejected {name}: {rc}")

    def forward(self, token: int, pos: int):
        rc = lib().gor_model_forward(self.m, int(token), int(pos))
        if rc != 0:
            raise RuntimeError("oracle forward: bad token/pos")

    def prefill(self, tokens, start_pos: int):
        for i, t in enumerate(tokens):
            self.forward(int(t), start_pos + i)

    def lm_head(self):
        lib().gor_model_lm_head(self.m)

    def select(self, temperature=0.0, top_p=0.9, rep_penalty=1.0, u=0.0, seen=()):
        s = np.ascontiguousarray(np.asarray(list(seen), dtype=np.int32))
        return lib().gor_model_select(self.m, temperature, top_p, rep_penalty, u,
                                      s.ctypes.data_as(_I32), len(s))

    def step(self, token, pos, **kw):
        self.forward(token, pos)
        return self.select(**kw)

    def reset_kv(self):
        lib().gor_model_reset_kv(self.m)

    def buffer(self, what: int, layer: int = 0) -> np.ndarray:
        s = self.shape
        n = {GOR_HIDDEN: s.hidden, GOR_NORMED: s.hidden, GOR_LOGITS: s.vocab, GOR_LAYER_HIDDEN: s.hidden,
             GOR_K_CACHE: s.ctx * s.kv_dim, GOR_V_CACHE: s.ctx * s.kv_dim, GOR_Q: s.q_dim,
             GOR_ATTN_OUT: s.q_dim}[what]
        p = lib().gor_model_buffer(self.m, what, layer)
        return np.ctypeslib.as_array(p, shape=(n,))

    def close(self):
        if self.m:
            lib().gor_model_destroy(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
