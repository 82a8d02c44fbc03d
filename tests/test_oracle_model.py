"""Pin the oracle's whole forward pass (engine.ts:735-802) against the
independent float64 restatement of debug.html's unfused forward pass, and
check mode / position properties of the token loop."""
from dataclasses import replace

import numpy as np
import pytest

from gemma_amd import synth
from oracle import oracle as orc

from f64_model import F64Model


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


@pytest.fixture(scope="module")
def tiny():
    shape = synth.TINY
    return shape, synth.make_model(shape, seed=7)


@pytest.mark.parametrize("mode", ["reference", "gemma3"])
def test_forward_matches_float64_statement(tiny, mode):
    shape, t = tiny
    shape = shape.reference_mode() if mode == "reference" else replace(shape.gemma3_mode(window=5))
    o = orc.OracleModel(shape, t)
    f = F64Model(shape, t)
    toks = synth.prompt_ids(12, seed=1, vocab=shape.vocab)
    for pos, tok in enumerate(toks):
        o.forward(int(tok), pos)
        f.forward(int(tok), pos)
        for l in range(shape.layers):
            assert rel(o.buffer(orc.GOR_LAYER_HIDDEN, l), f.hist[l]) < 1e-4, (pos, l)
        assert rel(o.buffer(orc.GOR_NORMED), f.normed) < 1e-4
    o.lm_head()
    assert rel(o.buffer(orc.GOR_LOGITS), f.logits()) < 1e-4


def test_embedding_row(tiny):
    shape, t = tiny
    for tok in (0, 5, shape.vocab - 1):
        e = orc.embed(t["token_embd.weight"][2], tok, shape.hidden)
        from gemma_amd.gguf import dequantize_q8_0_np
        row = dequantize_q8_0_np(t["token_embd.weight"][2], shape.vocab * shape.hidden).reshape(shape.vocab, -1)[tok]
        ref = (row * np.float32(np.sqrt(np.float32(shape.hidden)))).astype(np.float32)
        assert np.array_equal(e, ref)   # (q*d)*sqrt(H): two exact-then-rounded f32 products


def test_window_inert_below_its_length(tiny):
    # gemma3 mode with the local theta equal to the global one and window W
    # equals reference mode while pos < W, and differs after
    shape, t = tiny
    a = orc.OracleModel(shape.reference_mode(), t)
    b = orc.OracleModel(replace(shape.reference_mode(), window=6), t)
    toks = synth.prompt_ids(10, seed=2, vocab=shape.vocab)
    for pos, tok in enumerate(toks):
        a.forward(int(tok), pos)
        b.forward(int(tok), pos)
        same = np.array_equal(a.buffer(orc.GOR_NORMED), b.buffer(orc.GOR_NORMED))
        assert same == (pos < 6), pos


def test_multi_turn_positions_equal_single_run(tiny):
    # KV reuse: turns continue at kvPosition (engine.ts:988-990, 1030)
    shape, t = tiny
    toks = synth.prompt_ids(20, seed=3, vocab=shape.vocab)
    a = orc.OracleModel(shape, t)
    a.prefill(toks, 0)
    b = orc.OracleModel(shape, t)
    b.prefill(toks[:7], 0)
    b.prefill(toks[7:15], 7)
    b.prefill(toks[15:], 15)
    assert np.array_equal(a.buffer(orc.GOR_NORMED), b.buffer(orc.GOR_NORMED))


def test_select_paths(tiny):
    shape, t = tiny
    o = orc.OracleModel(shape, t)
    o.prefill(synth.prompt_ids(5, seed=4, vocab=shape.vocab), 0)
    g = o.select(0.0, 0.9, 1.0, 0.0)
    assert g == orc.argmax(o.buffer(orc.GOR_LOGITS))
    # T = 0 with a penalty goes through topk256 + sort
    v, i = orc.topk256(o.buffer(orc.GOR_LOGITS))
    assert o.select(0.0, 0.9, 1.2, 0.0, seen=[]) == int(i[np.argmax(v)])
