"""ctypes binding of libgg.so (include/gg.h) for Python callers: the tests,
the benchmark and __graft_entry__.

This is a thin mirror of the C-ABI; there is no compute in Python and no
fallback. If the HIP library is not built, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libgg.so")

GG_OK = 0
GG_ERR_INVALID = -1
GG_ERR_NO_DEVICE = -2
GG_ERR_HIP = -3
GG_ERR_DEVICE_LOST = -4
GG_ERR_MISSING = -5
GG_ERR_OOM = -6

GG_TYPE_F32 = 0
GG_TYPE_F16 = 1
GG_TYPE_Q8_0 = 8

GG_ATTN_REFERENCE = 0
GG_ATTN_GEMMA3 = 1

READ_HIDDEN = 0
READ_NORMED = 1
READ_LOGITS = 2
READ_TOPK256 = 3
READ_LAYER_HIDDEN = 4
READ_K_CACHE = 5
READ_V_CACHE = 6
READ_Q = 7
READ_ATTN_OUT = 8
READ_EMBED = 9

GG_DECODE_GRAPH = 0
GG_DECODE_FUSED = 1
DECODE_PATHS = {"graph": GG_DECODE_GRAPH, "fused": GG_DECODE_FUSED}

PROBE = {"none": 0, "qkv": 1, "attn": 2, "o": 3, "gate_up": 4, "down": 5, "lm_head": 6, "select": 7}


class GGConfig(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("context_length", ctypes.c_int32),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta_global", ctypes.c_float),
        ("rope_theta_local", ctypes.c_float),
        ("swa_period", ctypes.c_int32),
        ("sliding_window", ctypes.c_int32),
        ("attention_mode", ctypes.c_int32),
        ("prefill_batch", ctypes.c_int32),
    ]


class GGSample(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_double),
        ("top_p", ctypes.c_double),
        ("rep_penalty", ctypes.c_double),
    ]


class GGError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"gg error {code}: {msg}")
        self.code = code


_LIB = None

_P = ctypes.c_void_p
_SIGS = {
    "gg_create": (_P, [ctypes.POINTER(GGConfig)]),
    "gg_upload_tensor": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.c_uint32, _P, ctypes.c_size_t]),
    "gg_finalize": (ctypes.c_int, [_P]),
    "gg_prefill": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int32), ctypes.c_int32, ctypes.c_int32]),
    "gg_select": (ctypes.c_int, [_P, ctypes.POINTER(GGSample), ctypes.c_double, ctypes.POINTER(ctypes.c_int32)]),
    "gg_step": (ctypes.c_int, [_P, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(GGSample), ctypes.c_double,
                               ctypes.POINTER(ctypes.c_int32)]),
    "gg_step_submit": (ctypes.c_int, [_P, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(GGSample), ctypes.c_double]),
    "gg_step_collect": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int32)]),
    "gg_penalty_reset": (ctypes.c_int, [_P]),
    "gg_penalty_add": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int32), ctypes.c_int32]),
    "gg_reset_kv": (ctypes.c_int, [_P]),
    "gg_read": (ctypes.c_int, [_P, ctypes.c_int32, ctypes.c_int32, _P, ctypes.c_size_t]),
    "gg_set_timing": (ctypes.c_int, [_P, ctypes.c_int32]),
    "gg_last_timing": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]),
    "gg_set_probe": (ctypes.c_int, [_P, ctypes.c_int32, ctypes.c_int32]),
    "gg_probe_elapsed": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_float)]),
    "gg_probe_overhead": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_float)]),
    "gg_set_decode_path": (ctypes.c_int, [_P, ctypes.c_int32]),
    "gg_decode_path": (ctypes.c_int, [_P]),
    "gg_decode_timeline": (ctypes.c_int, [_P, _P, ctypes.c_size_t]),
    "gg_last_error": (ctypes.c_char_p, [_P]),
    "gg_destroy": (None, [_P]),
    "gg_q8_0_packed_size": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64]),
    "gg_q8_0_repack": (ctypes.c_int, [_P, _P, ctypes.c_int64, ctypes.c_int64, _P]),
    "gg_q8_0_gemv": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, ctypes.c_int64, _P]),
    "gg_q8_0_dequant": (ctypes.c_int, [_P, _P, ctypes.c_int64, _P]),
    "gg_select_workspace_size": (ctypes.c_size_t, [ctypes.c_int32]),
    "gg_select_logits": (ctypes.c_int, [_P, ctypes.c_int32, _P, ctypes.POINTER(GGSample), ctypes.c_double, _P, _P,
                                        ctypes.POINTER(ctypes.c_int32), _P]),
    "gg_select_logits_noalloc": (ctypes.c_int, [_P, ctypes.c_int32, _P, ctypes.POINTER(GGSample), ctypes.c_double,
                                                _P, ctypes.POINTER(ctypes.c_int32), _P]),
}


def lib() -> ctypes.CDLL:
    """Load libgg.so; raises if it has not been built (no fallback path)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
    return _LIB


def exported_symbols():
    return list(_SIGS)


def _check(ctx, rc):
    if rc != GG_OK:
        msg = lib().gg_last_error(ctx)
        raise GGError(rc, msg.decode() if msg else "")


def sample(temperature=0.0, top_p=0.9, rep_penalty=1.0) -> GGSample:
    return GGSample(float(temperature), float(top_p), float(rep_penalty))


class Engine:
    """One gg_ctx: weights, KV cache and the captured token graphs."""

    def __init__(self, cfg: GGConfig):
        L = lib()
        self._cfg = cfg
        self.ctx = L.gg_create(ctypes.byref(cfg))
        if not self.ctx:
            raise GGError(GG_ERR_INVALID, (L.gg_last_error(None) or b"").decode())

    @property
    def config(self) -> GGConfig:
        return self._cfg

    def upload(self, name: str, ggml_type: int, dims, data: np.ndarray):
        data = np.ascontiguousarray(data)
        d = (ctypes.c_uint64 * len(dims))(*[int(x) for x in dims])
        _check(self.ctx, lib().gg_upload_tensor(self.ctx, name.encode(), ggml_type, d, len(dims),
                                                data.ctypes.data, data.nbytes))

    def upload_model(self, tensors: dict):
        for name, (t, dims, data) in tensors.items():
            self.upload(name, t, dims, data)

    def set_decode_path(self, path: str):
        """"fused" (persistent kernel) or "graph" (one kernel per phase); before finalize()."""
        _check(self.ctx, lib().gg_set_decode_path(self.ctx, DECODE_PATHS[path]))

    def decode_path(self) -> str:
        rc = lib().gg_decode_path(self.ctx)
        if rc < 0:
            _check(self.ctx, rc)
        return "fused" if rc == GG_DECODE_FUSED else "graph"

    def decode_timeline(self) -> np.ndarray:
        """[256, layers, 16] s_memrealtime stamps of the last persistent-kernel launch."""
        out = np.zeros((256, self._cfg.num_layers, 16), dtype=np.int64)
        _check(self.ctx, lib().gg_decode_timeline(self.ctx, out.ctypes.data, out.size))
        return out

    def finalize(self):
        _check(self.ctx, lib().gg_finalize(self.ctx))

    def prefill(self, tokens, start_pos: int):
        arr = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        _check(self.ctx, lib().gg_prefill(self.ctx, arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                          len(arr), int(start_pos)))

    def select(self, temperature=0.0, top_p=0.9, rep_penalty=1.0, u=0.0) -> int:
        out = ctypes.c_int32(-1)
        s = sample(temperature, top_p, rep_penalty)
        _check(self.ctx, lib().gg_select(self.ctx, ctypes.byref(s), float(u), ctypes.byref(out)))
        return out.value

    def step(self, token: int, pos: int, temperature=0.0, top_p=0.9, rep_penalty=1.0, u=0.0) -> int:
        out = ctypes.c_int32(-1)
        s = sample(temperature, top_p, rep_penalty)
        _check(self.ctx, lib().gg_step(self.ctx, int(token), int(pos), ctypes.byref(s), float(u),
                                       ctypes.byref(out)))
        return out.value

    def step_submit(self, token: int, pos: int, temperature=0.0, top_p=0.9, rep_penalty=1.0, u=0.0):
        """Queue a step (token < 0: the id the previous step selects, on the device)."""
        s = sample(temperature, top_p, rep_penalty)
        _check(self.ctx, lib().gg_step_submit(self.ctx, int(token), int(pos), ctypes.byref(s), float(u)))

    def step_collect(self) -> int:
        """Wait for the oldest submitted step and return its id."""
        out = ctypes.c_int32(-1)
        _check(self.ctx, lib().gg_step_collect(self.ctx, ctypes.byref(out)))
        return out.value

    def penalty_reset(self):
        _check(self.ctx, lib().gg_penalty_reset(self.ctx))

    def penalty_add(self, ids):
        arr = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        _check(self.ctx, lib().gg_penalty_add(self.ctx, arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                              len(arr)))

    def reset_kv(self):
        _check(self.ctx, lib().gg_reset_kv(self.ctx))

    def read(self, what: int, layer: int = 0, count: int | None = None, dtype=np.float32) -> np.ndarray:
        c = self._cfg
        if count is None:
            count = {
                READ_HIDDEN: c.hidden_size, READ_NORMED: c.hidden_size, READ_LOGITS: c.vocab_size,
                READ_TOPK256: 512, READ_LAYER_HIDDEN: c.hidden_size,
                READ_K_CACHE: c.context_length * c.head_dim, READ_V_CACHE: c.context_length * c.head_dim,
                READ_Q: c.num_q_heads * c.head_dim, READ_ATTN_OUT: c.num_q_heads * c.head_dim,
                READ_EMBED: c.hidden_size,
            }[what]
        out = np.empty(count, dtype=dtype)
        _check(self.ctx, lib().gg_read(self.ctx, what, layer, out.ctypes.data, out.nbytes))
        return out

    def topk256(self):
        raw = self.read(READ_TOPK256, dtype=np.uint32)
        return raw[0::2].view(np.float32).copy(), raw[1::2].copy()

    def set_timing(self, on: bool):
        _check(self.ctx, lib().gg_set_timing(self.ctx, 1 if on else 0))

    def last_timing(self):
        a, b = ctypes.c_float(), ctypes.c_float()
        _check(self.ctx, lib().gg_last_timing(self.ctx, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def set_probe(self, kind: str, layer: int = 0):
        _check(self.ctx, lib().gg_set_probe(self.ctx, PROBE[kind], layer))

    def probe_elapsed_ms(self) -> float:
        v = ctypes.c_float()
        _check(self.ctx, lib().gg_probe_elapsed(self.ctx, ctypes.byref(v)))
        return v.value

    def probe_overhead_ms(self) -> float:
        """Device time of an empty event bracket recorded right before the probe."""
        v = ctypes.c_float()
        _check(self.ctx, lib().gg_probe_overhead(self.ctx, ctypes.byref(v)))
        return v.value

    def close(self):
        if self.ctx:
            lib().gg_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- kernel-level entry points (integer device pointers, stream handle) ----

def _stream_ptr(stream):
    if stream is None:
        return None
    return ctypes.c_void_p(int(stream))


def q8_0_repack(src_ptr: int, dst_ptr: int, rows: int, k: int, stream=None):
    _check(None, lib().gg_q8_0_repack(src_ptr, dst_ptr, rows, k, _stream_ptr(stream)))


def q8_0_packed_size(rows: int, k: int) -> int:
    return int(lib().gg_q8_0_packed_size(rows, k))


def q8_0_gemv(w_ptr: int, x_ptr: int, y_ptr: int, rows: int, k: int, stream=None):
    _check(None, lib().gg_q8_0_gemv(w_ptr, x_ptr, y_ptr, rows, k, _stream_ptr(stream)))


def q8_0_dequant(src_ptr: int, out_ptr: int, n: int, stream=None):
    _check(None, lib().gg_q8_0_dequant(src_ptr, out_ptr, n, _stream_ptr(stream)))


def select_workspace_size(n: int) -> int:
    return int(lib().gg_select_workspace_size(n))


def select_logits(logits_ptr: int, n: int, seen_ptr: int | None, temperature, top_p, rep_penalty, u,
                  ws_ptr: int, topk_ptr: int | None = None, stream=None) -> int:
    out = ctypes.c_int32(-1)
    s = sample(temperature, top_p, rep_penalty)
    _check(None, lib().gg_select_logits(logits_ptr, n, seen_ptr or None, ctypes.byref(s), float(u), ws_ptr,
                                        topk_ptr or None, ctypes.byref(out), _stream_ptr(stream)))
    return out.value


def select_logits_noalloc(logits_ptr: int, n: int, seen_ptr: int | None, temperature, top_p, rep_penalty, u,
                          topk_ptr: int | None = None, stream=None) -> int:
    """select_logits with the library's static per-device workspace (no device allocation)."""
    out = ctypes.c_int32(-1)
    s = sample(temperature, top_p, rep_penalty)
    _check(None, lib().gg_select_logits_noalloc(logits_ptr, n, seen_ptr or None, ctypes.byref(s), float(u),
                                                topk_ptr or None, ctypes.byref(out), _stream_ptr(stream)))
    return out.value
