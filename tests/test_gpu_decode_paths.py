"""The two decode paths through the C-ABI: the persistent kernel (one launch
per token, gg_decode.hip) and the per-kernel graph path compute the same
functions -- checked against each other at the full 1B shape and against
the oracle through the model tests -- plus the embedding row read back
bit-exact and the persistent kernel's timeout report."""
import os

import numpy as np
import pytest

from gemma_amd import capi, synth
from oracle import oracle as orc

from gpu_util import rel, say

pytestmark = pytest.mark.gpu


def engine(shape, tensors, path=None, prefill_batch=0):
    e = capi.Engine(shape.gg_config(prefill_batch=prefill_batch))
    if path:
        e.set_decode_path(path)
    e.upload_model(tensors)
    e.finalize()
    return e


@pytest.fixture(scope="module")
def tiny_model():
    return synth.make_model(synth.TINY, seed=7)


def test_decode_path_selection(gpu, tiny_model):
    """The persistent kernel is the default where its limits hold (4 query
    heads, hidden <= 1280, 256 CUs), at any context length: contexts above
    4096 run its long-span variant."""
    e = engine(synth.TINY.gemma3_mode(window=7), tiny_model)
    assert e.decode_path() == "fused"
    e.close()
    e = engine(synth.TINY.with_ctx(8192).gemma3_mode(window=7), tiny_model)
    assert e.decode_path() == "fused"
    e.close()
    e = engine(synth.TINY.gemma3_mode(window=7), tiny_model, "graph")
    assert e.decode_path() == "graph"
    e.close()


@pytest.mark.parametrize("path", ["fused", "graph"])
def test_sampled_steps_select_exactly_from_their_logits(gpu, path):
    """Sampling steps at the 270M shape (temperature 0.8, top-p 0.9,
    repetition penalty 1.3, a seeded draw u per step): each step's token is
    the oracle sampler's choice (engine.ts:862-901) over that step's own
    logits, read back after the step, with the turn's penalty set (prompt and
    every token chosen so far). On the persistent path the selection runs
    inside the step's launch."""
    shape = synth.GEMMA3_270M.with_ctx(1024).gemma3_mode()
    e = engine(shape, synth.make_model(shape, seed=5), path)
    assert e.decode_path() == path
    prompt = synth.prompt_ids(48, seed=7, vocab=shape.vocab)
    T, top_p, rep = 0.8, 0.9, 1.3
    rng = np.random.default_rng(11)
    e.penalty_reset()
    e.penalty_add(prompt)
    e.prefill(prompt, 0)
    seen = set(int(t) for t in prompt)
    tok = e.select(T, top_p, rep, float(rng.random()))
    seen.add(tok)
    pos = len(prompt)
    for step in range(24):
        u = float(rng.random())
        nxt = e.step(tok, pos, T, top_p, rep, u)
        vals, ids = orc.topk256(e.read(capi.READ_LOGITS))
        want = orc.sample_candidates(vals, ids, sorted(seen), T, top_p, rep, u)
        assert nxt == want, (path, step, nxt, want)
        seen.add(nxt)
        tok, pos = nxt, pos + 1
    e.close()


@pytest.mark.parametrize("shape_name", ["tiny", "270m"])
def test_embedding_row_bit_exact(gpu, tiny_model, shape_name):
    """embeddingLookup (shaders.ts:2-23): (f32(q) * scale) * sqrt(f32(H)) of the
    token's row, read through the device function both decode paths use,
    bit-exact against the oracle for tokens 0, 1, 106 and V - 1."""
    if shape_name == "tiny":
        shape, t = synth.TINY, tiny_model
    else:
        shape = synth.GEMMA3_270M.gemma3_mode()
        t = synth.make_model(shape, seed=270)
    e = engine(shape, t)
    emb = t["token_embd.weight"][2]
    for tok in (0, 1, 106, shape.vocab - 1):
        g = e.read(capi.READ_EMBED, tok)
        r = orc.embed(emb, tok, shape.hidden)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), f"token {tok}"
    e.close()


@pytest.mark.parametrize("mode", ["gemma3", "reference"])
def test_decode_paths_agree_1b(gpu, mode):
    """Full 1B shape at context 4096: both paths over the same 320-token
    prompt (token by token) and 24 greedy steps give the same tokens, every
    layer's hidden state and the logits within 1e-4, and the same K/V rows."""
    shape = synth.GEMMA3_1B.with_ctx(4096)
    shape = shape.gemma3_mode() if mode == "gemma3" else shape.reference_mode()
    say("1b paths build", mode)
    t = synth.make_model(shape, seed=3)
    prompt = synth.prompt_ids(320, seed=320, vocab=shape.vocab)
    runs = {}
    for path in ("fused", "graph"):
        e = engine(shape, t, path)
        assert e.decode_path() == path
        e.prefill(prompt, 0)
        tok = e.select()
        toks, hid, logits = [tok], [], []
        pos = len(prompt)
        for step in range(24):
            tok = e.step(tok, pos)
            toks.append(tok)
            pos += 1
            if step % 8 == 7:
                hid.append(np.stack([e.read(capi.READ_LAYER_HIDDEN, l) for l in range(shape.layers)]))
                logits.append(e.read(capi.READ_LOGITS))
        kv = [(e.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:pos],
               e.read(capi.READ_V_CACHE, l).reshape(shape.ctx, 256)[:pos]) for l in (0, 5, 11, 25)]
        runs[path] = (toks, hid, logits, kv)
        say("1b path", path, "tokens", toks[:6])
        e.close()
    (ta, ha, la, ka), (tb, hb, lb, kb) = runs["fused"], runs["graph"]
    assert ta == tb
    for x, y in zip(ha, hb):
        for l in range(shape.layers):
            assert rel(x[l], y[l]) < 1e-4, f"layer {l}"
    for x, y in zip(la, lb):
        assert rel(x, y) < 1e-4
    for (k1, v1), (k2, v2) in zip(ka, kb):
        assert rel(k1, k2) < 1e-4 and rel(v1, v2) < 1e-4


@pytest.mark.parametrize("mode", ["gemma3", "reference"])
def test_decode_paths_agree_1b_long_span(gpu, mode):
    """Full 1B shape at context 8192: a 4090-id prompt (batched prefill, the
    same K/V in both engines), then 24 greedy steps through positions
    4090..4113 on each path. The persistent kernel's full-attention layers
    switch from the 32-chunk layout to the 256-chunk four-head layout and its
    64-block merge at position 4096 (every layer in reference mode); the
    graph path runs its own long-span attention (k_attn_dec over 256 chunks
    + k_attn_merge). Same tokens, every layer's hidden state and the logits
    within 1e-4, the same K/V rows."""
    shape = synth.GEMMA3_1B.with_ctx(8192)
    shape = shape.gemma3_mode() if mode == "gemma3" else shape.reference_mode()
    say("1b long-span paths build", mode)
    t = synth.make_model(shape, seed=4)
    prompt = synth.prompt_ids(4090, seed=4090, vocab=shape.vocab)
    runs = {}
    for path in ("fused", "graph"):
        e = engine(shape, t, path, prefill_batch=2048)
        assert e.decode_path() == path
        e.prefill(prompt, 0)
        tok = e.select()
        toks, hid, logits = [tok], [], []
        pos = len(prompt)
        for step in range(24):
            tok = e.step(tok, pos)
            toks.append(tok)
            pos += 1
            if step in (4, 5, 6, 23):
                hid.append(np.stack([e.read(capi.READ_LAYER_HIDDEN, l) for l in range(shape.layers)]))
                logits.append(e.read(capi.READ_LOGITS))
        kv = [(e.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:pos],
               e.read(capi.READ_V_CACHE, l).reshape(shape.ctx, 256)[:pos]) for l in (0, 5, 11, 25)]
        runs[path] = (toks, hid, logits, kv)
        say("1b long-span path", path, "tokens", toks[:6])
        e.close()
    (ta, ha, la, ka), (tb, hb, lb, kb) = runs["fused"], runs["graph"]
    assert ta == tb
    for x, y in zip(ha, hb):
        for l in range(shape.layers):
            assert rel(x[l], y[l]) < 1e-4, f"layer {l}"
    for x, y in zip(la, lb):
        assert rel(x, y) < 1e-4
    for (k1, v1), (k2, v2) in zip(ka, kb):
        assert rel(k1, k2) < 1e-4 and rel(v1, v2) < 1e-4


@pytest.mark.parametrize("path", ["fused", "graph"])
def test_pipelined_steps_match_sequential_steps(gpu, path):
    """gg_step_submit / gg_step_collect with one step queued ahead, each next
    step taking its input id on the device (token -1), give the ids of
    sequential gg_step calls with the same draws: greedy, then sampled with a
    repetition penalty, at the 270M shape. Other calls are refused while a
    step is outstanding; a step queued past the last one is collected and
    dropped."""
    shape = synth.GEMMA3_270M.with_ctx(1024).gemma3_mode()
    t = synth.make_model(shape, seed=5)
    prompt = synth.prompt_ids(48, seed=48, vocab=shape.vocab)
    a, b = engine(shape, t, path), engine(shape, t, path)
    for opts in ((0.0, 0.9, 1.0), (0.8, 0.9, 1.3)):
        us = [float(x) for x in np.random.default_rng(3).random(25)]
        ids = {}
        for name, e in (("seq", a), ("pipe", b)):
            e.reset_kv()
            e.penalty_reset()
            e.penalty_add(prompt)
            e.prefill(prompt, 0)
            tok = e.select(*opts, us[0])
            out = [tok]
            if name == "seq":
                for k in range(24):
                    tok = e.step(tok, 48 + k, *opts, us[k + 1])
                    out.append(tok)
            else:
                e.step_submit(tok, 48, *opts, us[1])
                for k in range(24):
                    e.step_submit(-1, 48 + k + 1, *opts, us[min(k + 2, 24)])
                    out.append(e.step_collect())
                    if k == 3:
                        with pytest.raises(capi.GGError) as ex:
                            e.read(capi.READ_HIDDEN)
                        assert ex.value.code == capi.GG_ERR_INVALID
                e.step_collect()   # the step queued past the last one
            ids[name] = out
        assert ids["pipe"] == ids["seq"], opts
    a.close()
    b.close()


def test_persistent_kernel_timeout_is_reported(gpu, tiny_model, monkeypatch):
    """Every hand-off wait of the persistent kernel is bounded; a wait that
    runs out raises a host-visible flag and the block leaves, so the launch
    ends and the call reports a lost device. Forced from the host with a
    zero spin limit (the first unfinished poll gives up)."""
    monkeypatch.setenv("GG_DEC_SPIN_LIMIT", "0")
    shape = synth.TINY.gemma3_mode(window=7)
    e = engine(shape, tiny_model, "fused")
    monkeypatch.delenv("GG_DEC_SPIN_LIMIT")
    with pytest.raises(capi.GGError) as ex:
        for pos in range(4):
            e.step(5, pos)
    assert ex.value.code == capi.GG_ERR_DEVICE_LOST
    assert "persistent decode kernel" in str(ex.value)
    with pytest.raises(capi.GGError) as ex:
        e.step(5, 0)
    assert ex.value.code == capi.GG_ERR_DEVICE_LOST
    e.close()
    # a fresh context works
    e = engine(shape, tiny_model, "fused")
    e.step(5, 0)
    e.close()
