"""Writes the tiny-model golden vectors: tests/golden/tiny_<mode>.npz.

The 2-layer TINY Gemma-3 shape (hidden 128, 4 query heads of 256, 1 KV head,
FFN 256, vocab 2048) with seeded Q8_0 weights (synth.make_model, seed 7) runs a
9-token seeded prompt and 12 greedy tokens through tests/f64_model.py, the
float64 statement of the reference's unfused debug pass (debug.html:1983-2087).
Stored: per-layer hidden, normed hidden and logits after the prompt, and the
greedy ids. A sha256 of the weight bytes guards against generator drift.

Run from the repo root: python tests/golden/make_tiny_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "webgpu-gemma_amd"), os.path.dirname(HERE)]

from gemma_amd import synth  # noqa: E402
from f64_model import F64Model  # noqa: E402

MODES = {"reference": synth.TINY.reference_mode(), "gemma3": synth.TINY.gemma3_mode(window=7)}
SEED, PROMPT_SEED, N_PROMPT, N_GEN = 7, 11, 9, 12


def weights_digest(tensors) -> str:
    h = hashlib.sha256()
    for name in sorted(tensors):
        h.update(name.encode())
        h.update(np.ascontiguousarray(tensors[name][2]).tobytes())
    return h.hexdigest()


def golden(shape, tensors):
    m = F64Model(shape, tensors)
    prompt = synth.prompt_ids(N_PROMPT, seed=PROMPT_SEED, vocab=shape.vocab)
    for p, t in enumerate(prompt):
        m.forward(int(t), p)
    out = {"prompt": prompt.astype(np.int32), "hist": m.hist.copy(), "normed": m.normed.copy(),
           "logits": m.logits()}
    toks, pos = [], len(prompt)
    tok = int(np.argmax(out["logits"]))
    for _ in range(N_GEN):
        toks.append(tok)
        m.forward(tok, pos)
        pos += 1
        tok = int(np.argmax(m.logits()))
    out["greedy"] = np.array(toks, np.int32)
    return out


def main():
    tensors = synth.make_model(synth.TINY, seed=SEED)
    digest = weights_digest(tensors)
    for mode, shape in MODES.items():
        g = golden(shape, tensors)
        np.savez_compressed(os.path.join(HERE, f"tiny_{mode}.npz"), weights_sha256=np.array(digest), **g)
        print(mode, "greedy", g["greedy"].tolist())


if __name__ == "__main__":
    main()
