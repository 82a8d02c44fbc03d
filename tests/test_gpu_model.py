"""Whole token loop on the GPU through the C-ABI against the oracle:
per-layer hidden states, normed hidden and logits within 1e-3 relative,
identical greedy and sampled token sequences, and the position/KV-reuse
properties of the reference's generate() loop (engine.ts:957-1031)."""
from dataclasses import replace

import numpy as np
import pytest

from gemma_amd import capi, synth
from oracle import oracle as orc

from gpu_util import rel, say

pytestmark = pytest.mark.gpu

TOL = 1e-3
_MODELS = {}


def engine(shape, tensors, path=None):
    e = capi.Engine(shape.gg_config())
    if path:
        e.set_decode_path(path)
    e.upload_model(tensors)
    e.finalize()
    if path:
        assert e.decode_path() == path
    return e


def check_state(e, o, shape, what=""):
    for l in range(shape.layers):
        r = rel(e.read(capi.READ_LAYER_HIDDEN, l), o.buffer(orc.GOR_LAYER_HIDDEN, l))
        assert r < TOL, f"{what} layer {l} hidden rel {r:.2e}"
    r = rel(e.read(capi.READ_NORMED), o.buffer(orc.GOR_NORMED))
    assert r < TOL, f"{what} normed rel {r:.2e}"


@pytest.fixture(scope="module")
def tiny_model():
    return synth.make_model(synth.TINY, seed=7)


@pytest.mark.parametrize("path", ["fused", "graph"])
@pytest.mark.parametrize("mode", ["reference", "gemma3"])
def test_tiny_greedy_loop(gpu, tiny_model, mode, path):
    shape = synth.TINY.reference_mode() if mode == "reference" else synth.TINY.gemma3_mode(window=7)
    say("tiny greedy", mode, path)
    e = engine(shape, tiny_model, path)
    o = orc.OracleModel(shape, tiny_model)
    prompt = synth.prompt_ids(9, seed=11, vocab=shape.vocab)
    e.prefill(prompt, 0)
    o.prefill(prompt, 0)
    check_state(e, o, shape, "prefill")
    tok = e.select(0.0, 0.9, 1.0, 0.0)
    assert tok == o.select(0.0, 0.9, 1.0, 0.0)
    assert rel(e.read(capi.READ_LOGITS), o.buffer(orc.GOR_LOGITS)) < TOL
    pos = len(prompt)
    for step in range(24):
        nxt = e.step(tok, pos, 0.0, 0.9, 1.0, 0.0)
        o.forward(tok, pos)
        ref = o.select(0.0, 0.9, 1.0, 0.0)
        check_state(e, o, shape, f"step {step}")
        assert rel(e.read(capi.READ_LOGITS), o.buffer(orc.GOR_LOGITS)) < TOL
        assert nxt == ref, f"step {step}"
        tok, pos = nxt, pos + 1
    # the KV cache rows written so far match
    for l in range(shape.layers):
        kc = e.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:pos]
        vc = e.read(capi.READ_V_CACHE, l).reshape(shape.ctx, 256)[:pos]
        assert rel(kc, o.buffer(orc.GOR_K_CACHE, l).reshape(shape.ctx, 256)[:pos]) < TOL
        assert rel(vc, o.buffer(orc.GOR_V_CACHE, l).reshape(shape.ctx, 256)[:pos]) < TOL
    e.close()


@pytest.mark.parametrize("path", ["fused", "graph"])
def test_tiny_context_filled_to_its_last_position(gpu, tiny_model, path):
    """The last positions of the context: a batched prefill of ctx - 6 ids,
    then greedy steps at ctx - 6 .. ctx - 1 (the last cache row) against the
    oracle, every K/V row of the full cache compared; then, after a reset, one
    batched prefill that ends exactly at ctx (engine.ts:923-928 allows
    start + n == contextLength)."""
    shape = synth.TINY.gemma3_mode(window=7)
    ctx = shape.ctx
    say("tiny context to its last position", path)
    e = capi.Engine(shape.gg_config(prefill_batch=64))
    e.set_decode_path(path)
    e.upload_model(tiny_model)
    e.finalize()
    assert e.decode_path() == path
    o = orc.OracleModel(shape, tiny_model)
    prompt = synth.prompt_ids(ctx - 6, seed=13, vocab=shape.vocab)
    e.prefill(prompt, 0)
    o.prefill(prompt, 0)
    tok = e.select(0.0, 0.9, 1.0, 0.0)
    assert tok == o.select(0.0, 0.9, 1.0, 0.0)
    pos = len(prompt)
    while pos < ctx:
        nxt = e.step(tok, pos, 0.0, 0.9, 1.0, 0.0)
        o.forward(tok, pos)
        ref = o.select(0.0, 0.9, 1.0, 0.0)   # the oracle's LM head runs in its select
        check_state(e, o, shape, f"pos {pos}")
        assert rel(e.read(capi.READ_LOGITS), o.buffer(orc.GOR_LOGITS)) < TOL, pos
        assert nxt == ref, pos
        tok, pos = nxt, pos + 1
    for l in range(shape.layers):
        assert rel(e.read(capi.READ_K_CACHE, l), o.buffer(orc.GOR_K_CACHE, l)) < TOL, l
        assert rel(e.read(capi.READ_V_CACHE, l), o.buffer(orc.GOR_V_CACHE, l)) < TOL, l
    with pytest.raises(capi.GGError):
        e.step(tok, ctx)
    full = synth.prompt_ids(ctx, seed=14, vocab=shape.vocab)
    e.reset_kv()
    e.prefill(full, 0)
    o2 = orc.OracleModel(shape, tiny_model)
    o2.prefill(full, 0)
    check_state(e, o2, shape, "prefill to ctx")
    assert e.select(0.0, 0.9, 1.0, 0.0) == o2.select(0.0, 0.9, 1.0, 0.0)
    e.close()


def test_prefill_equals_steps_and_turns(gpu, tiny_model):
    shape = synth.TINY.gemma3_mode(window=5)
    say("prefill vs steps")
    toks = synth.prompt_ids(17, seed=12, vocab=shape.vocab)
    a = engine(shape, tiny_model)
    a.prefill(toks, 0)
    b = engine(shape, tiny_model)
    for i, t in enumerate(toks):        # one token per call, positions 0..16
        b.prefill([t], i)
    c = engine(shape, tiny_model)       # three turns continuing at kvPosition
    c.prefill(toks[:4], 0)
    c.prefill(toks[4:11], 4)
    c.prefill(toks[11:], 11)
    ref = a.read(capi.READ_NORMED)
    assert np.array_equal(b.read(capi.READ_NORMED), ref)
    assert np.array_equal(c.read(capi.READ_NORMED), ref)
    for l in range(shape.layers):
        assert np.array_equal(b.read(capi.READ_K_CACHE, l), a.read(capi.READ_K_CACHE, l))
    # reset_kv + re-prefill reproduces the same state
    a.reset_kv()
    a.prefill(toks, 0)
    assert np.array_equal(a.read(capi.READ_NORMED), ref)
    for x in (a, b, c):
        x.close()


def test_tiny_sampling_stream(gpu, tiny_model):
    # temperature / top-p / repetition penalty with an injected uniform stream
    shape = synth.TINY.gemma3_mode(window=6)
    say("tiny sampling")
    e = engine(shape, tiny_model)
    o = orc.OracleModel(shape, tiny_model)
    rng = np.random.default_rng(5)
    prompt = list(synth.prompt_ids(8, seed=13, vocab=shape.vocab))
    e.penalty_reset()
    e.penalty_add(prompt)
    e.prefill(prompt, 0)
    o.prefill(prompt, 0)
    seen = list(prompt)
    opts = (0.7, 0.9, 1.2)
    u = float(rng.random())
    tok = e.select(*opts, u)
    assert tok == o.select(*opts, u, seen=seen)
    seen.append(tok)
    pos = len(prompt)
    for step in range(30):
        u = float(rng.random())
        nxt = e.step(tok, pos, *opts, u)
        o.forward(tok, pos)
        assert nxt == o.select(*opts, u, seen=seen), f"step {step}"
        seen.append(nxt)
        tok, pos = nxt, pos + 1
    e.close()


@pytest.mark.parametrize("path", ["fused", "graph"])
def test_270m_greedy_128(gpu, path):
    """270M architecture, gemma3 mode: 64 seeded prompt ids then 128 greedy
    tokens, identical to the oracle; logits within 1e-3 at checkpoints."""
    shape = synth.GEMMA3_270M.gemma3_mode()
    say("270m build", path)
    t = synth.make_model(shape, seed=270)
    e = engine(shape, t, path)
    o = orc.OracleModel(shape, t)
    prompt = synth.prompt_ids(64, seed=64, vocab=shape.vocab)
    e.prefill(prompt, 0)
    o.prefill(prompt, 0)
    check_state(e, o, shape, "prefill")
    tok = e.select()
    assert tok == o.select()
    gpu_toks, ref_toks = [tok], [tok]
    pos = 64
    for step in range(127):
        nxt = e.step(tok, pos)
        o.forward(tok, pos)
        ref = o.select()
        if step % 32 == 0:
            say("270m step", step)
            check_state(e, o, shape, f"step {step}")
            assert rel(e.read(capi.READ_LOGITS), o.buffer(orc.GOR_LOGITS)) < TOL
        gpu_toks.append(nxt)
        ref_toks.append(ref)
        assert nxt == ref, f"token {step + 1} differs"
        tok, pos = nxt, pos + 1
    assert len(gpu_toks) == 128
    e.close()


@pytest.mark.parametrize("mode,ctx,span", [("gemma3", 4096, 2048), ("reference", 4096, 2048),
                                           ("gemma3", 32768, 32768 - 8)])
def test_1b_full_size_step_with_shared_kv(gpu, mode, ctx, span):
    """Gemma-3-1B shapes at full size: fill the KV cache on the GPU (step by
    step prefill of `span` seeded ids), copy it into the oracle, then compare
    one decode step (per-layer hidden, logits, greedy id) at that position."""
    shape = synth.GEMMA3_1B.with_ctx(ctx)
    shape = shape.gemma3_mode() if mode == "gemma3" else shape.reference_mode()
    say("1b build", mode, ctx, span)
    if "1b" not in _MODELS:
        _MODELS["1b"] = synth.make_model(shape, seed=1)
    t = _MODELS["1b"]
    e = engine(shape, t)
    prompt = synth.prompt_ids(span, seed=2048, vocab=shape.vocab)
    e.prefill(prompt, 0)
    say("1b prefilled")
    o = orc.OracleModel(shape, t)
    for l in range(shape.layers):
        o.buffer(orc.GOR_K_CACHE, l)[:] = e.read(capi.READ_K_CACHE, l)
        o.buffer(orc.GOR_V_CACHE, l)[:] = e.read(capi.READ_V_CACHE, l)
    tok = int(prompt[-1])
    nxt = e.step(tok, span, 0.0, 0.9, 1.0, 0.0)
    o.forward(tok, span)
    ref = o.select(0.0, 0.9, 1.0, 0.0)
    check_state(e, o, shape, "1b step")
    assert rel(e.read(capi.READ_LOGITS), o.buffer(orc.GOR_LOGITS)) < TOL
    assert nxt == ref
    e.close()


@pytest.mark.parametrize("mode", ["reference", "gemma3"])
def test_tiny_gpu_matches_golden(gpu, tiny_model, mode):
    """The GPU path against the committed float64 golden vectors
    (tests/golden/tiny_<mode>.npz): per-layer hidden, normed and logits after
    the prompt within 1e-4, and the same 12 greedy ids."""
    import os
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", f"tiny_{mode}.npz"),
                allow_pickle=False)
    shape = synth.TINY.reference_mode() if mode == "reference" else synth.TINY.gemma3_mode(window=7)
    e = engine(shape, tiny_model)
    e.prefill(g["prompt"], 0)
    for l in range(shape.layers):
        assert rel(e.read(capi.READ_LAYER_HIDDEN, l), g["hist"][l]) < 1e-4, l
    assert rel(e.read(capi.READ_NORMED), g["normed"]) < 1e-4
    tok = e.select()
    assert rel(e.read(capi.READ_LOGITS), g["logits"]) < 1e-4
    toks, pos = [], len(g["prompt"])
    for _ in range(len(g["greedy"])):
        toks.append(tok)
        tok = e.step(tok, pos)
        pos += 1
    assert toks == g["greedy"].tolist()
    e.close()


def test_1b_32k_three_turns_sampling(gpu):
    """Gemma-3-1B at contextLength 32768, gemma3 attention: three chained turns
    whose prompts fill ~32K positions of KV, sampling with T=0.7, topP=0.9,
    rep=1.2 and a seeded u stream (generate(), engine.ts:957-1031: per-turn
    penalty set = the turn's prompt + its generated ids; the last generated id
    of a turn is not written to the KV cache).
    * every sampled id equals the reference's selection (topk256 + host
      sampler, engine.ts:854-901, in the oracle) on the GPU's own logits;
    * KV reuse: a second engine that prefills every id the first one wrote
      (one call) and then takes the same last step reproduces its logits and
      id bit for bit."""
    shape = synth.GEMMA3_1B.with_ctx(32768).gemma3_mode()
    if "1b" not in _MODELS:
        _MODELS["1b"] = synth.make_model(shape, seed=1)
    t = _MODELS["1b"]
    e = engine(shape, t)
    rng = np.random.default_rng(55)
    opts = (0.7, 0.9, 1.2)
    prompts = [synth.prompt_ids(n, seed=300 + i, vocab=shape.vocab) for i, n in enumerate([16384, 8192, 8100])]
    kv_ids, kv_pos = [], 0
    last = None
    for turn, p in enumerate(prompts):
        say("32k turn", turn, "prefill", len(p), "at", kv_pos)
        e.penalty_reset()
        e.penalty_add(p)
        e.prefill(p, kv_pos)
        kv_ids += [int(x) for x in p]
        kv_pos += len(p)
        seen = [int(x) for x in p]
        u = float(rng.random())
        tok = e.select(*opts, u)
        vals, ids = orc.topk256(e.read(capi.READ_LOGITS))
        assert tok == orc.sample_candidates(vals, ids, seen, *opts, u), f"turn {turn} first id"
        seen.append(tok)
        writes = 0
        for k in range(7):
            pos = kv_pos + writes
            u = float(rng.random())
            nxt = e.step(tok, pos, *opts, u)
            kv_ids.append(tok)
            writes += 1
            logits = e.read(capi.READ_LOGITS)
            vals, ids = orc.topk256(logits)
            assert nxt == orc.sample_candidates(vals, ids, seen, *opts, u), f"turn {turn} step {k}"
            seen.append(nxt)
            last = (tok, pos, u, seen[:-1], logits, nxt)
            tok = nxt
        kv_pos += writes
    assert kv_pos == len(kv_ids) and kv_pos < shape.ctx - 10
    e.close()
    # KV reuse: one prefill of everything but the last written id, then that step
    say("32k replay", len(kv_ids) - 1)
    b = engine(shape, t)
    b.penalty_reset()
    b.penalty_add(last[3])
    b.prefill(kv_ids[:-1], 0)
    tok, pos, u, _, logits, nxt = last
    assert b.step(tok, pos, *opts, u) == nxt
    assert np.array_equal(b.read(capi.READ_LOGITS), logits)
    b.close()


def test_step_timing_opt_in_and_fused_final(gpu, tiny_model):
    """gg_set_timing: gg_last_timing fails while timing is off and returns the
    step's device times while it is on. The timed step runs the forward graph
    with k_final and the plain LM head; the untimed step runs the step graph,
    whose LM head prologue does k_final's work: both give the same logits,
    hidden state and tokens bit for bit."""
    shape = synth.TINY.gemma3_mode(window=7)
    say("step timing + fused final norm")
    a, b = engine(shape, tiny_model), engine(shape, tiny_model)
    prompt = synth.prompt_ids(9, seed=11, vocab=shape.vocab)
    for e in (a, b):
        e.prefill(prompt, 0)
    ta, tb = a.select(), b.select()
    assert ta == tb
    b.set_timing(True)
    pos = len(prompt)
    for step in range(6):
        ta = a.step(ta, pos)
        with pytest.raises(capi.GGError):
            a.last_timing()
        tb = b.step(tb, pos)
        fwd, sel = b.last_timing()
        assert fwd > 0.0 and sel > 0.0
        assert ta == tb, f"step {step}"
        for what in (capi.READ_LOGITS, capi.READ_HIDDEN, capi.READ_NORMED):
            assert np.array_equal(a.read(what), b.read(what)), f"step {step} read {what}"
        pos += 1
    b.set_timing(False)
    tb = b.step(tb, pos)
    with pytest.raises(capi.GGError):
        b.last_timing()
    a.close()
    b.close()
