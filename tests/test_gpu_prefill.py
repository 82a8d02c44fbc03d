"""Batched prefill (M-row GEMMs on bf16 MFMA + MFMA flash attention) against the
oracle's token-by-token prefill (engine.ts:923-928) and against the GPU's own
per-token path at the Gemma-3-1B shape."""
import numpy as np
import pytest

from gemma_amd import capi, synth
from oracle import oracle as orc

from gpu_util import rel, say

pytestmark = pytest.mark.gpu
TOL = 1e-3
_MODELS = {}


def engine(shape, tensors, batch):
    e = capi.Engine(shape.gg_config(prefill_batch=batch))
    e.upload_model(tensors)
    e.finalize()
    return e


@pytest.fixture(scope="module")
def tiny_model():
    return synth.make_model(synth.TINY, seed=7)


@pytest.mark.parametrize("mode,batch,n", [("reference", 64, 40), ("gemma3", 64, 40), ("gemma3", 16, 53),
                                          ("gemma3", 256, 200)])
def test_tiny_batched_prefill_matches_oracle(gpu, tiny_model, mode, batch, n):
    shape = synth.TINY.reference_mode() if mode == "reference" else synth.TINY.gemma3_mode(window=9)
    say("tiny batched prefill", mode, batch, n)
    e = engine(shape, tiny_model, batch)
    o = orc.OracleModel(shape, tiny_model)
    prompt = synth.prompt_ids(n, seed=21, vocab=shape.vocab)
    e.prefill(prompt, 0)
    o.prefill(prompt, 0)
    for l in range(shape.layers):
        assert rel(e.read(capi.READ_LAYER_HIDDEN, l), o.buffer(orc.GOR_LAYER_HIDDEN, l)) < TOL, l
        kc = e.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:n]
        vc = e.read(capi.READ_V_CACHE, l).reshape(shape.ctx, 256)[:n]
        assert rel(kc, o.buffer(orc.GOR_K_CACHE, l).reshape(shape.ctx, 256)[:n]) < TOL, l
        assert rel(vc, o.buffer(orc.GOR_V_CACHE, l).reshape(shape.ctx, 256)[:n]) < TOL, l
    assert rel(e.read(capi.READ_NORMED), o.buffer(orc.GOR_NORMED)) < TOL
    tok = e.select()
    assert tok == o.select()
    # decode continues from the batched prefill exactly like from the oracle's
    pos = n
    for _ in range(6):
        nxt = e.step(tok, pos)
        o.forward(tok, pos)
        assert nxt == o.select()
        tok, pos = nxt, pos + 1
    e.close()


def test_tiny_second_turn_batched(gpu, tiny_model):
    # a second prefill continues at kvPosition (engine.ts:988-990)
    shape = synth.TINY.gemma3_mode(window=7)
    e = engine(shape, tiny_model, 32)
    o = orc.OracleModel(shape, tiny_model)
    a = synth.prompt_ids(20, seed=1, vocab=shape.vocab)
    b = synth.prompt_ids(15, seed=2, vocab=shape.vocab)
    e.prefill(a, 0)
    e.prefill(b, 20)
    o.prefill(a, 0)
    o.prefill(b, 20)
    assert rel(e.read(capi.READ_NORMED), o.buffer(orc.GOR_NORMED)) < TOL
    assert e.select() == o.select()
    e.close()


@pytest.mark.parametrize("mode", ["gemma3", "reference"])
def test_1b_batched_prefill_2048_matches_token_by_token(gpu, mode):
    shape = synth.GEMMA3_1B.with_ctx(4096)
    shape = shape.gemma3_mode() if mode == "gemma3" else shape.reference_mode()
    say("1b batched prefill", mode)
    if "1b" not in _MODELS:
        _MODELS["1b"] = synth.make_model(shape, seed=1)
    t = _MODELS["1b"]
    prompt = synth.prompt_ids(2048, seed=2048, vocab=shape.vocab)
    a = engine(shape, t, 2048)
    a.prefill(prompt, 0)
    b = engine(shape, t, 0)
    b.prefill(prompt, 0)
    say("1b prefilled both")
    for l in range(shape.layers):
        assert rel(a.read(capi.READ_LAYER_HIDDEN, l), b.read(capi.READ_LAYER_HIDDEN, l)) < TOL, l
    for l in (0, 5, 13, 25):
        assert rel(a.read(capi.READ_K_CACHE, l), b.read(capi.READ_K_CACHE, l)) < TOL, l
        assert rel(a.read(capi.READ_V_CACHE, l), b.read(capi.READ_V_CACHE, l)) < TOL, l
    ta, tb = a.select(), b.select()
    assert rel(a.read(capi.READ_LOGITS), b.read(capi.READ_LOGITS)) < TOL
    assert ta == tb
    pos = 2048
    for _ in range(8):
        ta, tb = a.step(ta, pos), b.step(tb, pos)
        assert ta == tb
        pos += 1
    a.close()
    b.close()


def test_1b_batched_prefill_short_turns_match_token_by_token(gpu):
    """Gemma-3-1B shapes, gemma3 attention: two short turns (300 prompt ids,
    then 77 more at position 300) batched against the token-by-token path.
    Row counts this small run the QKV, O and down GEMMs on 96-wide tiles
    (K split in 2 and 4), the 2048-row prefill only its QKV GEMM."""
    shape = synth.GEMMA3_1B.with_ctx(4096).gemma3_mode()
    say("1b short batched turns, 300 + 77 ids")
    if "1b" not in _MODELS:
        _MODELS["1b"] = synth.make_model(shape, seed=1)
    t = _MODELS["1b"]
    first = synth.prompt_ids(300, seed=300, vocab=shape.vocab)
    second = synth.prompt_ids(77, seed=77, vocab=shape.vocab)
    a = engine(shape, t, 2048)
    b = engine(shape, t, 0)
    pos = 0
    for ids in (first, second):
        a.prefill(ids, pos)
        b.prefill(ids, pos)
        pos += len(ids)
        for l in range(shape.layers):
            assert rel(a.read(capi.READ_LAYER_HIDDEN, l), b.read(capi.READ_LAYER_HIDDEN, l)) < TOL, (pos, l)
        for l in (0, 5, 25):
            ka = a.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:pos]
            kb = b.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:pos]
            assert rel(ka, kb) < TOL, (pos, l)
        ta, tb = a.select(), b.select()
        assert rel(a.read(capi.READ_LOGITS), b.read(capi.READ_LOGITS)) < TOL, pos
        assert ta == tb, pos
    for _ in range(4):
        ta, tb = a.step(ta, pos), b.step(tb, pos)
        assert ta == tb
        pos += 1
    a.close()
    b.close()


def test_1b_batched_prefill_ragged_slices_long_span(gpu):
    """Gemma-3-1B shapes at contextLength 8192, gemma3 attention: a 6000-id
    prompt prefilled in ragged batched slices (2500 + 2500 + 1000 rows: no
    slice length or start is a multiple of the 128-row GEMM tile, and the
    global layers' key spans reach 6000) against the token-by-token path;
    then decode steps past 4096 positions (256-chunk attention + merge)."""
    shape = synth.GEMMA3_1B.with_ctx(8192).gemma3_mode()
    say("1b ragged batched prefill, 6000 ids")
    if "1b" not in _MODELS:
        _MODELS["1b"] = synth.make_model(shape, seed=1)
    t = _MODELS["1b"]
    prompt = synth.prompt_ids(6000, seed=6000, vocab=shape.vocab)
    a = engine(shape, t, 2500)
    a.prefill(prompt, 0)
    b = engine(shape, t, 0)
    b.prefill(prompt, 0)
    say("1b prefilled both")
    for l in range(shape.layers):
        assert rel(a.read(capi.READ_LAYER_HIDDEN, l), b.read(capi.READ_LAYER_HIDDEN, l)) < TOL, l
    for l in (0, 5, 11, 25):
        ka = a.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:6000]
        kb = b.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:6000]
        assert rel(ka, kb) < TOL, l
    ta, tb = a.select(), b.select()
    assert rel(a.read(capi.READ_LOGITS), b.read(capi.READ_LOGITS)) < TOL
    assert ta == tb
    pos = 6000
    for _ in range(6):
        ta, tb = a.step(ta, pos), b.step(tb, pos)
        assert ta == tb
        pos += 1
    a.close()
    b.close()


def test_1b_batched_prefill_32k_matches_token_path_and_oracle(gpu):
    """Gemma-3-1B at contextLength 32768, gemma3 attention: a 32760-id prompt
    prefilled in batched slices of 4096 rows (the global layers' prefill
    attention over key spans up to 32760) against the token-by-token path on
    the persistent kernel: every layer's hidden state, the normed hidden and
    the K/V rows of the global layers 5, 11, 17 and 23 over all 32760
    positions. Then the oracle takes the batched engine's K/V cache and both
    run 8 greedy steps from position 32760: per-layer hidden, logits and ids
    against the oracle at every step."""
    shape = synth.GEMMA3_1B.with_ctx(32768).gemma3_mode()
    n = 32760
    say("1b 32k batched prefill vs token path")
    if "1b" not in _MODELS:
        _MODELS["1b"] = synth.make_model(shape, seed=1)
    t = _MODELS["1b"]
    prompt = synth.prompt_ids(n, seed=32760, vocab=shape.vocab)
    a = engine(shape, t, 4096)
    a.prefill(prompt, 0)
    b = engine(shape, t, 0)
    b.prefill(prompt, 0)
    say("1b 32k prefilled both")
    for l in range(shape.layers):
        assert rel(a.read(capi.READ_LAYER_HIDDEN, l), b.read(capi.READ_LAYER_HIDDEN, l)) < TOL, l
    assert rel(a.read(capi.READ_NORMED), b.read(capi.READ_NORMED)) < TOL
    for l in (5, 11, 17, 23):
        for what in (capi.READ_K_CACHE, capi.READ_V_CACHE):
            ka = a.read(what, l).reshape(shape.ctx, 256)[:n]
            kb = b.read(what, l).reshape(shape.ctx, 256)[:n]
            assert rel(ka, kb) < TOL, (l, what)
    b.close()
    o = orc.OracleModel(shape, t)
    for l in range(shape.layers):
        o.buffer(orc.GOR_K_CACHE, l)[:] = a.read(capi.READ_K_CACHE, l)
        o.buffer(orc.GOR_V_CACHE, l)[:] = a.read(capi.READ_V_CACHE, l)
    tok, pos = int(prompt[-1]), n - 1
    # the prompt's last row again as a decode step (the same K/V row), then 8 steps
    for step in range(9):
        nxt = a.step(tok, pos)
        o.forward(tok, pos)
        ref = o.select()
        for l in range(shape.layers):
            assert rel(a.read(capi.READ_LAYER_HIDDEN, l), o.buffer(orc.GOR_LAYER_HIDDEN, l)) < TOL, (step, l)
        assert rel(a.read(capi.READ_LOGITS), o.buffer(orc.GOR_LOGITS)) < TOL, step
        assert nxt == ref, f"step {step}"
        say("1b 32k step", step, nxt)
        tok, pos = nxt, pos + 1
    o.close()
    a.close()


def test_270m_batched_prefill_matches_oracle(gpu):
    """Gemma-3-270M architecture (hidden 640: 128-wide GEMM tiles with a K
    split, 64-row prompt), gemma3 attention: the 64-id prompt in one batched
    prefill against the oracle's token-by-token prefill (per-layer hidden,
    K/V cache, normed hidden), then 32 greedy tokens identical to it."""
    shape = synth.GEMMA3_270M.gemma3_mode()
    say("270m batched prefill")
    t = synth.make_model(shape, seed=270)
    e = engine(shape, t, 64)
    o = orc.OracleModel(shape, t)
    prompt = synth.prompt_ids(64, seed=64, vocab=shape.vocab)
    e.prefill(prompt, 0)
    o.prefill(prompt, 0)
    for l in range(shape.layers):
        assert rel(e.read(capi.READ_LAYER_HIDDEN, l), o.buffer(orc.GOR_LAYER_HIDDEN, l)) < TOL, l
    for l in (0, 5, 17):
        kc = e.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:64]
        assert rel(kc, o.buffer(orc.GOR_K_CACHE, l).reshape(shape.ctx, 256)[:64]) < TOL, l
    assert rel(e.read(capi.READ_NORMED), o.buffer(orc.GOR_NORMED)) < TOL
    tok = e.select()
    assert tok == o.select()
    pos = 64
    for step in range(32):
        nxt = e.step(tok, pos)
        o.forward(tok, pos)
        assert nxt == o.select(), f"step {step}"
        tok, pos = nxt, pos + 1
    e.close()
