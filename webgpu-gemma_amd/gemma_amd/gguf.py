"""GGUF v3 container and the Q8_0 / F16 formats the token loop reads.

Mirrors the reference's reader (src/gguf.ts): little-endian header, typed
key/value metadata, tensor infos, data section aligned to 32 bytes
(gguf.ts:67-93); Q8_0 = 34-byte blocks of an f16 scale and 32 int8
(gguf.ts:107-124, 181-187). The writer produces files that reader accepts.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

GGUF_MAGIC = 0x46554747
ALIGN = 32

T_F32, T_F16, T_Q8_0 = 0, 1, 8

# metadata value types (gguf.ts:42-65)
V_UINT8, V_INT8, V_UINT16, V_INT16, V_UINT32, V_INT32, V_FLOAT32, V_BOOL, V_STRING, V_ARRAY, V_UINT64, V_INT64, \
    V_FLOAT64 = range(13)

_SCALAR = {V_UINT8: "<B", V_INT8: "<b", V_UINT16: "<H", V_INT16: "<h", V_UINT32: "<I", V_INT32: "<i",
           V_FLOAT32: "<f", V_BOOL: "<?", V_UINT64: "<Q", V_INT64: "<q", V_FLOAT64: "<d"}


def tensor_nbytes(ggml_type: int, n_elems: int) -> int:
    """gguf.ts:181-187."""
    if ggml_type == T_Q8_0:
        return n_elems // 32 * 34
    if ggml_type == T_F32:
        return n_elems * 4
    if ggml_type == T_F16:
        return n_elems * 2
    raise ValueError(f"unknown tensor type {ggml_type}")


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """Q8_0 blocks of a float array whose size is a multiple of 32:
    d = max|w| / 127 stored as f16, q = round(w / d) clamped to [-127, 127]."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1, 32)
    amax = np.abs(w).max(axis=1)
    d = amax / np.float32(127.0)
    inv = np.zeros_like(d)
    nz = d > 0
    inv[nz] = np.float32(1.0) / d[nz]
    q = np.rint(w * inv[:, None])
    np.clip(q, -127, 127, out=q)
    out = np.empty((w.shape[0], 34), dtype=np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def q8_0_blocks(scales_f16: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Assemble Q8_0 bytes from explicit f16 scales [nb] and int8 quants [nb, 32]."""
    nb = scales_f16.shape[0]
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, :2] = np.ascontiguousarray(scales_f16, dtype=np.float16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = np.ascontiguousarray(q, dtype=np.int8).reshape(nb, 32).view(np.uint8)
    return out.reshape(-1)


def dequantize_q8_0_np(blocks: np.ndarray, n: int) -> np.ndarray:
    """Reference semantics of dequantizeQ8_0 (q * scale, exact in f32)."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 34)[: n // 32]
    d = b[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (q * d).reshape(-1)


@dataclass
class TensorInfo:
    name: str
    dims: list
    ggml_type: int
    offset: int

    @property
    def n_elems(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n

    @property
    def nbytes(self) -> int:
        return tensor_nbytes(self.ggml_type, self.n_elems)


def _w_str(buf: list, s: str):
    b = s.encode("utf-8")
    buf.append(struct.pack("<Q", len(b)))
    buf.append(b)


def _w_value(buf: list, vtype: int, v):
    if vtype in _SCALAR:
        buf.append(struct.pack(_SCALAR[vtype], v))
    elif vtype == V_STRING:
        _w_str(buf, v)
    elif vtype == V_ARRAY:
        etype, items = v
        buf.append(struct.pack("<IQ", etype, len(items)))
        if etype == V_STRING:
            for it in items:
                _w_str(buf, it)
        else:
            buf.append(np.asarray(items, dtype=np.dtype(_SCALAR[etype])).tobytes())
    else:
        raise ValueError(f"unsupported metadata type {vtype}")


def write_gguf(path: str, kv: list, tensors: list):
    """kv: [(key, vtype, value)]; tensors: [(name, ggml_type, dims, bytes ndarray)]."""
    head = [struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(kv))]
    for key, vtype, value in kv:
        _w_str(head, key)
        head.append(struct.pack("<I", vtype))
        _w_value(head, vtype, value)
    offset = 0
    offsets = []
    for name, t, dims, data in tensors:
        _w_str(head, name)
        head.append(struct.pack("<I", len(dims)))
        for d in dims:
            head.append(struct.pack("<Q", int(d)))
        head.append(struct.pack("<IQ", t, offset))
        offsets.append(offset)
        offset += (data.nbytes + ALIGN - 1) // ALIGN * ALIGN
    header = b"".join(head)
    pad = (-len(header)) % ALIGN
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * pad)
        for (name, t, dims, data), off in zip(tensors, offsets):
            raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
            f.write(raw.tobytes())
            f.write(b"\0" * ((-raw.nbytes) % ALIGN))


class GGUFFile:
    """Memory-mapped GGUF reader (gguf.ts:67-93 + getTensorData*)."""

    def __init__(self, path: str):
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        self.off = 0
        magic, self.version = struct.unpack_from("<II", self.mm, 0)
        if magic != GGUF_MAGIC:
            raise ValueError(f"Invalid GGUF magic: 0x{magic:x}")
        n_t, n_kv = struct.unpack_from("<QQ", self.mm, 8)
        self.off = 24
        self.kv = {}
        for _ in range(n_kv):
            key = self._r_str()
            (vt,) = struct.unpack_from("<I", self.mm, self.off)
            self.off += 4
            self.kv[key] = self._r_value(vt)
        self.tensors = []
        for _ in range(n_t):
            name = self._r_str()
            (nd,) = struct.unpack_from("<I", self.mm, self.off)
            self.off += 4
            dims = list(struct.unpack_from(f"<{nd}Q", self.mm, self.off))
            self.off += 8 * nd
            t, o = struct.unpack_from("<IQ", self.mm, self.off)
            self.off += 12
            self.tensors.append(TensorInfo(name, dims, t, o))
        self.data_offset = (self.off + ALIGN - 1) // ALIGN * ALIGN

    def _r_str(self) -> str:
        (n,) = struct.unpack_from("<Q", self.mm, self.off)
        self.off += 8
        s = bytes(self.mm[self.off:self.off + n]).decode("utf-8")
        self.off += n
        return s

    def _r_value(self, vt: int):
        if vt in _SCALAR:
            fmt = _SCALAR[vt]
            (v,) = struct.unpack_from(fmt, self.mm, self.off)
            self.off += struct.calcsize(fmt)
            return v
        if vt == V_STRING:
            return self._r_str()
        if vt == V_ARRAY:
            et, n = struct.unpack_from("<IQ", self.mm, self.off)
            self.off += 12
            return [self._r_value(et) for _ in range(n)]
        raise ValueError(f"unknown metadata type {vt}")

    def tensor(self, name: str) -> TensorInfo:
        for t in self.tensors:
            if t.name == name:
                return t
        raise KeyError(name)

    def tensor_bytes(self, t: TensorInfo) -> np.ndarray:
        start = self.data_offset + t.offset
        return self.mm[start:start + t.nbytes]
