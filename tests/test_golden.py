"""The C oracle against the committed tiny-model golden vectors
(tests/golden/tiny_<mode>.npz, written by tests/golden/make_tiny_golden.py
from the float64 statement of the reference's unfused debug pass)."""
import os

import numpy as np
import pytest

from gemma_amd import synth
from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODES = {"reference": synth.TINY.reference_mode(), "gemma3": synth.TINY.gemma3_mode(window=7)}


def load(mode):
    return np.load(os.path.join(GOLDEN, f"tiny_{mode}.npz"), allow_pickle=False)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.fixture(scope="module")
def tensors():
    return synth.make_model(synth.TINY, seed=7)


def test_generator_matches_the_fixture(tensors):
    from golden.make_tiny_golden import weights_digest
    for mode in MODES:
        assert str(load(mode)["weights_sha256"]) == weights_digest(tensors)


@pytest.mark.parametrize("mode", list(MODES))
def test_oracle_matches_golden(tensors, mode):
    g = load(mode)
    shape = MODES[mode]
    o = orc.OracleModel(shape, tensors)
    o.prefill(g["prompt"], 0)
    for l in range(shape.layers):
        assert rel(o.buffer(orc.GOR_LAYER_HIDDEN, l), g["hist"][l]) < 1e-5, l
    assert rel(o.buffer(orc.GOR_NORMED), g["normed"]) < 1e-5
    o.lm_head()
    assert rel(o.buffer(orc.GOR_LOGITS), g["logits"]) < 1e-5
    tok, pos, toks = o.select(), len(g["prompt"]), []
    for _ in range(len(g["greedy"])):
        toks.append(tok)
        o.forward(tok, pos)
        pos += 1
        tok = o.select()
    assert toks == g["greedy"].tolist()
    o.close()
