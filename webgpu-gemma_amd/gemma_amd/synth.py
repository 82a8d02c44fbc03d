"""Seeded random-init Gemma-3 models and GEMV operands for the token loop.

Shapes follow the Gemma-3 270M / 1B GGUF files the reference loads
(src/types.ts:19-36 defaults; gguf.ts:190-220 metadata). Weights are
Q8_0 of N(0, 0.02): per 32 weights d = max|w|/127 stored as f16 and
q = round(w/d) in [-127, 127]. Norm weights are 1 + 0.1 N(0, 1) in f32
(GGUF Gemma norms already include the +1).
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np

from . import capi
from .gguf import T_F32, T_Q8_0, V_ARRAY, V_FLOAT32, V_STRING, V_UINT32, quantize_q8_0, q8_0_blocks, write_gguf

Q8_NAMES = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
NORM_NAMES = ["attn_norm", "ffn_norm", "attn_q_norm", "attn_k_norm", "post_attention_norm", "post_ffw_norm"]


@dataclass(frozen=True)
class Shape:
    hidden: int
    layers: int
    n_q: int
    inter: int
    vocab: int = 262144
    ctx: int = 2048
    head_dim: int = 256
    n_kv: int = 1
    eps: float = 1e-6
    theta_global: float = 1e6
    theta_local: float = 1e6
    swa_period: int = 6
    window: int = 0

    @property
    def q_dim(self):
        return self.n_q * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv * self.head_dim

    def gemma3_mode(self, window=512, theta_local=1e4) -> "Shape":
        """Local layers: theta 1e4, sliding window 512 (Gemma-3 as published)."""
        return replace(self, window=window, theta_local=theta_local)

    def reference_mode(self) -> "Shape":
        """src/ as shipped: theta 1e6 on every layer, full attention."""
        return replace(self, window=0, theta_local=self.theta_global)

    def with_ctx(self, ctx: int) -> "Shape":
        return replace(self, ctx=ctx)

    def gg_config(self, prefill_batch: int = 0) -> capi.GGConfig:
        return capi.GGConfig(self.hidden, self.layers, self.n_q, self.n_kv, self.head_dim, self.inter, self.vocab,
                             self.ctx, self.eps, self.theta_global, self.theta_local, self.swa_period, self.window,
                             capi.GG_ATTN_GEMMA3 if self.window else capi.GG_ATTN_REFERENCE, prefill_batch)

    def weight_count(self) -> int:
        per_layer = self.hidden * (self.q_dim + 2 * self.kv_dim) + self.q_dim * self.hidden + 3 * self.hidden * self.inter
        return self.vocab * self.hidden + self.layers * per_layer

    def q8_bytes(self) -> int:
        return self.weight_count() // 32 * 34


GEMMA3_270M = Shape(hidden=640, layers=18, n_q=4, inter=2048)
GEMMA3_1B = Shape(hidden=1152, layers=26, n_q=4, inter=6912)
TINY = Shape(hidden=128, layers=2, n_q=4, inter=256, vocab=2048, ctx=256)


def _q8(rng: np.random.Generator, rows: int, k: int, std: float = 0.02) -> np.ndarray:
    w = rng.standard_normal(rows * k, dtype=np.float32)
    w *= np.float32(std)
    return quantize_q8_0(w)


def make_model(shape: Shape, seed: int = 0) -> dict:
    """{gguf name: (ggml_type, dims, bytes)}; dims[0] is the input dimension."""
    rng = np.random.default_rng(seed)
    H, I, Q, KV = shape.hidden, shape.inter, shape.q_dim, shape.kv_dim
    t = {"token_embd.weight": (T_Q8_0, [H, shape.vocab], _q8(rng, shape.vocab, H))}
    t["output_norm.weight"] = (T_F32, [H], (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    dims = {"attn_q": (H, Q), "attn_k": (H, KV), "attn_v": (H, KV), "attn_output": (Q, H),
            "ffn_gate": (H, I), "ffn_up": (H, I), "ffn_down": (I, H)}
    for l in range(shape.layers):
        for n in Q8_NAMES:
            k, rows = dims[n]
            t[f"blk.{l}.{n}.weight"] = (T_Q8_0, [k, rows], _q8(rng, rows, k))
        for n in NORM_NAMES:
            size = shape.head_dim if n in ("attn_q_norm", "attn_k_norm") else H
            t[f"blk.{l}.{n}.weight"] = (T_F32, [size], (1.0 + 0.1 * rng.standard_normal(size)).astype(np.float32))
    return t


def prompt_ids(n: int, seed: int, vocab: int) -> np.ndarray:
    """Seeded uniform token ids in [0, vocab)."""
    return np.random.default_rng(seed).integers(0, vocab, size=n, dtype=np.int64).astype(np.int32)


def gemv_operands(rows: int, k: int, seed: int):
    """Isolated GEMV operands: q uniform in [-127, 127], |d| = exp(N(-6, 0.5))
    as f16 with a random sign, x ~ N(0, 1) in f32."""
    rng = np.random.default_rng(seed)
    nb = rows * k // 32
    q = rng.integers(-127, 128, size=(nb, 32), dtype=np.int32).astype(np.int8)
    d = np.exp(rng.normal(-6.0, 0.5, size=nb)) * rng.choice([-1.0, 1.0], size=nb)
    blocks = q8_0_blocks(d.astype(np.float16), q)
    x = rng.standard_normal(k).astype(np.float32)
    return blocks, x


def synthetic_vocab(vocab: int) -> list:
    """Token strings with the reference's special ids (tokenizer.ts:3-8)."""
    toks = [f"<unused{i}>" for i in range(vocab)]
    special = {0: "<pad>", 1: "<eos>", 2: "<bos>", 3: "<unk>", 105: "<start_of_turn>", 106: "<end_of_turn>"}
    for i, s in special.items():
        if i < vocab:
            toks[i] = s
    base = ["▁", "a", "b", "c", "d", "e", "\n", "user", "model", "▁the", "▁a", "Hello", "?", "."]
    for j, s in enumerate(base):
        if 200 + j < vocab:
            toks[200 + j] = s
    return toks


def write_model_gguf(path: str, shape: Shape, seed: int = 0, tensors: dict | None = None,
                     rope_base_swa: float | None = None):
    """A GGUF the reference parser accepts (gguf.ts:190-220 keys), plus the
    rope frequency base Gemma-3 files carry (shape.theta_global) and, when
    given, a sliding-window layer base."""
    tensors = tensors if tensors is not None else make_model(shape, seed)
    kv = [
        ("general.architecture", V_STRING, "gemma3"),
        ("gemma3.embedding_length", V_UINT32, shape.hidden),
        ("gemma3.block_count", V_UINT32, shape.layers),
        ("gemma3.feed_forward_length", V_UINT32, shape.inter),
        ("gemma3.attention.head_count", V_UINT32, shape.n_q),
        ("gemma3.attention.head_count_kv", V_UINT32, shape.n_kv),
        ("gemma3.attention.key_length", V_UINT32, shape.head_dim),
        ("gemma3.context_length", V_UINT32, max(shape.ctx, 32768)),
        ("gemma3.attention.sliding_window", V_UINT32, 512),
        ("gemma3.rope.freq_base", V_FLOAT32, float(shape.theta_global)),
        ("tokenizer.ggml.tokens", V_ARRAY, (V_STRING, synthetic_vocab(shape.vocab))),
    ]
    if rope_base_swa is not None:
        kv.append(("gemma3.rope.freq_base_swa", V_FLOAT32, float(rope_base_swa)))
    write_gguf(path, kv, [(n, t, d, b) for n, (t, d, b) in tensors.items()])
