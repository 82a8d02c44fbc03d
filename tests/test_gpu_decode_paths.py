"""The two decode paths through the C-ABI: the persistent kernel (one launch
per token, gg_decode.hip) and the per-kernel graph path compute the same
functions -- checked against each other at the full 1B shape and against
the oracle through the model tests -- plus the embedding row read back
bit-exact and the persistent kernel's fallback to the graph path when a
hand-off wait runs out."""
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
    # the ends of the draw and of the top-p cutoff: u = 0 and just below 1,
    # top-p 1 (possibly all 256 candidates), a top-p below the first
    # probability, a near-flat distribution at a high temperature
    top = 1.0 - 2.0 ** -40
    for T, top_p, rep, u in [(0.8, 0.9, 1.3, 0.0), (0.8, 0.9, 1.3, top), (0.8, 1.0, 1.3, float(rng.random())),
                             (0.8, 1.0, 1.0, top), (0.8, 1e-6, 1.3, float(rng.random())),
                             (50.0, 0.999, 1.3, float(rng.random())), (50.0, 1.0, 1.0, top)]:
        nxt = e.step(tok, pos, T, top_p, rep, u)
        vals, ids = orc.topk256(e.read(capi.READ_LOGITS))
        want = orc.sample_candidates(vals, ids, sorted(seen), T, top_p, rep, u)
        assert nxt == want, (path, T, top_p, rep, u, nxt, want)
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


def test_persistent_kernel_timeout_falls_back_to_graphs(gpu, monkeypatch):
    """Every hand-off wait of the persistent kernel is bounded: a launch whose
    wait runs out raises its flags in mapped host memory and ends. The context
    then drains its stream, clears the hand-off words and carries on on the
    graph path, running the timed-out work again there: a token-by-token
    prefill and synchronous steps (engine a), and pipelined steps -- the one
    that timed out and the one queued behind it, which took its id on the
    device (engine b). Both give the graph path's ids and K/V rows. Forced
    from the host with a zero spin limit (the first poll that finds its words
    missing gives up); the vocabulary is a multiple of 16384 so that a step
    is one launch."""
    shape = synth.Shape(hidden=128, layers=2, n_q=4, inter=256, vocab=16384, ctx=256).gemma3_mode(window=7)
    t = synth.make_model(shape, seed=7)
    prompt = synth.prompt_ids(9, seed=11, vocab=shape.vocab)
    ref_a, ref_b = engine(shape, t, "graph"), engine(shape, t, "graph", prefill_batch=16)
    monkeypatch.setenv("GG_DEC_SPIN_LIMIT", "0")
    a, b = engine(shape, t, "fused"), engine(shape, t, "fused", prefill_batch=16)
    monkeypatch.delenv("GG_DEC_SPIN_LIMIT")
    assert a.decode_path() == "fused" and b.decode_path() == "fused"

    def run_sync(e):
        e.prefill(prompt, 0)
        tok = e.select()
        ids, pos = [tok], len(prompt)
        for _ in range(6):
            tok = e.step(tok, pos)
            ids.append(tok)
            pos += 1
        return ids

    def run_pipelined(e):
        e.prefill(prompt, 0)   # batched: no persistent launch
        tok = e.select()
        ids, pos = [tok], len(prompt)
        e.step_submit(tok, pos)
        for k in range(6):
            if k < 5:
                e.step_submit(-1, pos + 1)
            ids.append(e.step_collect())
            pos += 1
        return ids

    say("timeout fallback: synchronous")
    assert run_sync(a) == run_sync(ref_a)
    assert a.decode_path() == "graph"
    say("timeout fallback: pipelined")
    assert run_pipelined(b) == run_pipelined(ref_b)
    assert b.decode_path() == "graph"
    n = len(prompt) + 6
    for e, r in ((a, ref_a), (b, ref_b)):
        for l in range(shape.layers):
            for what in (capi.READ_K_CACHE, capi.READ_V_CACHE):
                got = e.read(what, l).reshape(shape.ctx, 256)[:n]
                want = r.read(what, l).reshape(shape.ctx, 256)[:n]
                assert rel(got, want) < 1e-4, (l, what)
    for e in (a, b, ref_a, ref_b):
        e.close()
    # a fresh context runs on the persistent kernel again
    e = engine(shape, t, "fused")
    e.step(5, 0)
    assert e.decode_path() == "fused"
    e.close()


def _brev8(c):
    return int(f"{c:08b}"[::-1], 2)


def test_fused_step_ties_follow_the_reference_rule(gpu):
    """Exact ties on the persistent step's LM head and selection
    (shaders.ts:327-384). A model's tied embedding copies the row t* that
    wins a greedy step into rows of t*'s own stride class (lower and higher
    indices: the same lane in an earlier / later row group of the same wave,
    another wave's group, a neighbouring lane) and into rows of the classes
    whose 8-bit bit-reversed ids lie just below and just above t*'s; with an
    unchanged hidden state their logits equal t*'s bit for bit, the maximum.
    The fused class candidates and block 0's selection must then give
    orc.argmax of the read-back logits (the bit-reversed class rule, then the
    first index; also checked against that rule in closed form),
    GG_READ_TOPK256 must equal orc.topk256, and sampled steps (T 0.7, top-p
    0.9, repetition 1.2, three draws) must pick orc.sample_candidates' id."""
    shape = synth.Shape(hidden=128, layers=2, n_q=4, inter=256, vocab=262144, ctx=256).gemma3_mode(window=7)
    t = synth.make_model(shape, seed=21)
    prompt = synth.prompt_ids(9, seed=5, vocab=shape.vocab)
    pos = len(prompt)
    e = engine(shape, t, "fused")
    e.prefill(prompt, 0)
    tok0 = e.select()
    e.step(tok0, pos)
    L = e.read(capi.READ_LOGITS)
    e.close()
    ts = int(np.argmax(L))
    c, k = ts % 256, ts // 256          # class, index inside the class (lane k % 64, row group k // 64)
    rows = set()
    for dk in (-256, -64, -1, 1, 64, 256, -512, 512):
        if 0 <= k + dk < shape.vocab // 256:
            rows.add(c + 256 * (k + dk))
    rng = np.random.default_rng(3)
    for db in (-1, 1):                  # classes whose bit-reversed id is just below / above t*'s
        b = _brev8(c) + db
        if 0 <= b < 256:
            rows.add(_brev8(b) + 256 * int(rng.integers(0, shape.vocab // 256)))
    rows -= set(int(x) for x in prompt) | {tok0, ts}
    assert len(rows) >= 6
    emb = t["token_embd.weight"][2].reshape(shape.vocab, -1).copy()
    for r in rows:
        emb[r] = emb[ts]
    t2 = dict(t)
    t2["token_embd.weight"] = (t["token_embd.weight"][0], t["token_embd.weight"][1], emb.reshape(-1))
    e = engine(shape, t2, "fused")
    assert e.decode_path() == "fused"
    say("ties", ts, sorted(rows))

    e.prefill(prompt, 0)
    e.select()
    g = e.step(tok0, pos)                # greedy
    L2 = e.read(capi.READ_LOGITS)
    tied = np.nonzero(L2 == L2.max())[0]
    assert set(int(i) for i in tied) == rows | {ts}, "the copied rows are the tied maxima"
    from test_oracle_kernels import closed_form_argmax
    assert g == orc.argmax(L2) == closed_form_argmax(L2)
    vals, ids = orc.topk256(L2)
    top = e.read(capi.READ_TOPK256).view(np.uint32).reshape(256, 2)
    assert np.array_equal(top[:, 0], vals.view(np.uint32)) and np.array_equal(top[:, 1], ids)

    seen = sorted(set(int(x) for x in prompt) | {tok0})
    for u in (0.02, 0.5, 0.97):
        e.prefill(prompt, 0)
        e.select()
        e.penalty_reset()
        e.penalty_add(np.array(seen, np.int32))
        s = e.step(tok0, pos, 0.7, 0.9, 1.2, u)
        L3 = e.read(capi.READ_LOGITS)
        assert np.array_equal(L3.view(np.uint32), L2.view(np.uint32))
        v3, i3 = orc.topk256(L3)
        assert s == orc.sample_candidates(v3, i3, seen, 0.7, 0.9, 1.2, u), u
    e.close()


@pytest.mark.parametrize("switch", ["GG_DEC_COOP", "GG_DEC_TIMELINE", "GG_NO_GRAPH"])
def test_launch_switches_leave_results_unchanged(gpu, monkeypatch, switch):
    """The launch switches a context reads at finalize change how kernels are
    launched or observed, not what they compute: a cooperative launch of the
    persistent kernel (GG_DEC_COOP=1), its phase stamps (GG_DEC_TIMELINE=1)
    and direct launches instead of graphs (GG_NO_GRAPH=1) give the same
    batched prefill, the same greedy and sampled ids and the same final
    hidden state, bit for bit, as the default context on the 270M shape."""
    shape = synth.GEMMA3_270M.with_ctx(1024).gemma3_mode()
    tensors = synth.make_model(shape, seed=3)
    prompt = synth.prompt_ids(100, seed=5, vocab=shape.vocab)

    def run():
        e = engine(shape, tensors, prefill_batch=64)
        assert e.decode_path() == "fused"
        e.prefill(prompt, 0)
        tok = e.select()
        ids, pos = [tok], len(prompt)
        for i in range(12):
            if i % 2:
                tok = e.step(tok, pos, 0.8, 0.9, 1.3, 0.1 * i)
            else:
                tok = e.step(tok, pos)
            ids.append(tok)
            pos += 1
        hidden = e.read(capi.READ_HIDDEN).copy()
        e.close()
        return ids, hidden

    want_ids, want_hidden = run()
    monkeypatch.setenv(switch, "1")
    say(f"{switch}=1")
    got_ids, got_hidden = run()
    monkeypatch.delenv(switch)
    assert got_ids == want_ids, (switch, got_ids, want_ids)
    assert np.array_equal(got_hidden, want_hidden), (switch, rel(got_hidden, want_hidden))


def test_profiling_probes_and_timeline(gpu, monkeypatch):
    """The profiling entry points report plausible device times and stamps
    without changing what a step computes: on the graph path a probe on one
    layer's gate/up GEMV (gg_set_probe) gives an elapsed time below the
    step's own forward time (an empty bracket of its own is reported beside
    it), with the same ids as an unprobed context; on the persistent path
    GG_DEC_TIMELINE=1 fills every (block, layer) start stamp
    (gg_decode_timeline), in increasing layer order within each block."""
    shape = synth.GEMMA3_270M.with_ctx(1024).gemma3_mode()
    tensors = synth.make_model(shape, seed=4)
    prompt = synth.prompt_ids(40, seed=6, vocab=shape.vocab)

    def steps(e, n=6):
        e.prefill(prompt, 0)
        tok = e.select()
        ids, pos = [tok], len(prompt)
        for _ in range(n):
            tok = e.step(tok, pos)
            ids.append(tok)
            pos += 1
        return ids

    plain = engine(shape, tensors, "graph")
    want = steps(plain)
    plain.close()

    e = capi.Engine(shape.gg_config())
    e.set_decode_path("graph")
    e.set_probe("gate_up", 3)
    e.upload_model(tensors)
    e.finalize()
    e.set_timing(True)
    assert steps(e) == want
    elapsed, overhead = e.probe_elapsed_ms(), e.probe_overhead_ms()
    fwd_ms, _ = e.last_timing()
    say(f"probe {elapsed * 1e3:.2f} us, bracket {overhead * 1e3:.2f} us, forward {fwd_ms * 1e3:.1f} us")
    # on direct launches the empty bracket can span a host dispatch gap, so
    # only the probed launch is bounded by the forward time
    assert 0.0 < elapsed < fwd_ms and overhead >= 0.0, (overhead, elapsed, fwd_ms)
    e.close()

    monkeypatch.setenv("GG_DEC_TIMELINE", "1")
    e = engine(shape, tensors)
    monkeypatch.delenv("GG_DEC_TIMELINE")
    assert e.decode_path() == "fused"
    steps(e, 2)
    tl = e.decode_timeline()
    e.close()
    assert tl.shape == (256, shape.layers, 16)
    start = tl[:, :, 0]
    assert (start > 0).all()
    assert (np.diff(start, axis=1) > 0).all()


def test_invalid_calls_are_refused_and_leave_the_context_usable(gpu, tiny_model):
    """Arguments and call orders the C-ABI refuses: each returns its error
    code (GG_ERR_INVALID, or GG_ERR_MISSING for an incomplete model) and
    changes nothing, so the same context then prefills and decodes exactly
    as a fresh one (the reference throws for the same misuse and keeps the
    engine, engine.ts:923-1031)."""
    shape = synth.TINY.gemma3_mode(window=7)
    V, L, ctx = shape.vocab, shape.layers, shape.gg_config().context_length
    prompt = synth.prompt_ids(9, seed=11, vocab=V)

    def refused(code, fn, *args, **kw):
        with pytest.raises(capi.GGError) as ex:
            fn(*args, **kw)
        assert ex.value.code == code, (fn.__name__, ex.value.code, str(ex.value))

    fresh = engine(shape, tiny_model, prefill_batch=4)
    fresh.prefill(prompt, 0)
    want = [fresh.select()]
    for k in range(5):
        want.append(fresh.step(want[-1], len(prompt) + k))
    fresh.close()

    e = engine(shape, tiny_model, prefill_batch=4)
    inv = capi.GG_ERR_INVALID
    refused(inv, e.step_submit, -1, 0)                        # no id selected yet
    refused(inv, e.step_collect)                              # nothing outstanding
    refused(inv, e.prefill, [0, V], 0)                        # token id out of range
    refused(inv, e.prefill, prompt, ctx - 3)                  # range past the context
    refused(inv, e.read, 99, count=4)                         # unknown target
    refused(inv, e.read, capi.READ_LAYER_HIDDEN, layer=L)     # layer out of range
    refused(inv, e.set_decode_path, "graph")                  # after finalize
    refused(inv, e.set_probe, "qkv", 0)                       # after finalize
    refused(inv, e.probe_elapsed_ms)                          # no probe set
    refused(inv, e.decode_timeline)                           # no timeline requested
    refused(inv, e.last_timing)                               # timing off
    refused(inv, e.upload, "output_norm.weight", 0, [shape.hidden], np.ones(shape.hidden, np.float32))
    e.prefill(prompt, 0)
    got = [e.select()]
    refused(inv, e.step, got[0], ctx)                         # position outside the context
    refused(inv, e.step, V, len(prompt))                      # token out of range
    e.step_submit(got[0], len(prompt))
    e.step_submit(-1, len(prompt) + 1)
    refused(inv, e.step_submit, -1, len(prompt) + 2)          # two steps outstanding
    refused(inv, e.read, capi.READ_HIDDEN)                    # state busy while steps are queued
    got += [e.step_collect(), e.step_collect()]
    for k in range(2, 5):
        got.append(e.step(got[-1], len(prompt) + k))
    assert got == want, (got, want)
    e.close()

    partial = capi.Engine(shape.gg_config())
    refused(capi.GG_ERR_MISSING, partial.finalize)            # no tensors uploaded
    partial.close()


def test_two_persistent_contexts_take_turns(gpu):
    """Two contexts of one process on one device, each on the persistent
    kernel, interleave their steps (sequential and pipelined, with steps of
    both queued at once): their launches take turns, so neither times out
    and falls back to the graph path, and each produces exactly the ids it
    produces alone."""
    shape = synth.GEMMA3_270M.with_ctx(1024).gemma3_mode()
    ta, tb = synth.make_model(shape, seed=21), synth.make_model(shape, seed=22)
    pa = synth.prompt_ids(30, seed=1, vocab=shape.vocab)
    pb = synth.prompt_ids(45, seed=2, vocab=shape.vocab)

    def alone(t, prompt):
        e = engine(shape, t, prefill_batch=32)
        e.prefill(prompt, 0)
        ids = [e.select()]
        for k in range(16):
            ids.append(e.step(ids[-1], len(prompt) + k))
        e.close()
        return ids

    want_a, want_b = alone(ta, pa), alone(tb, pb)
    a, b = engine(shape, ta, prefill_batch=32), engine(shape, tb, prefill_batch=32)
    assert a.decode_path() == b.decode_path() == "fused"
    a.prefill(pa, 0)
    b.prefill(pb, 0)
    ga, gb = [a.select()], [b.select()]
    for k in range(8):   # sequential, alternating
        ga.append(a.step(ga[-1], len(pa) + k))
        gb.append(b.step(gb[-1], len(pb) + k))
    a.step_submit(ga[-1], len(pa) + 8)
    b.step_submit(gb[-1], len(pb) + 8)
    for k in range(9, 16):   # pipelined on both, one step of each queued ahead
        a.step_submit(-1, len(pa) + k)
        b.step_submit(-1, len(pb) + k)
        ga.append(a.step_collect())
        gb.append(b.step_collect())
    ga.append(a.step_collect())
    gb.append(b.step_collect())
    assert a.decode_path() == b.decode_path() == "fused"
    assert ga == want_a, (ga, want_a)
    assert gb == want_b, (gb, want_b)
    a.close()
    b.close()


def test_two_persistent_contexts_from_two_threads(gpu):
    """The same two contexts driven from two host threads at once (the
    binding runs its calls on a thread pool; ctypes releases the GIL around
    each C call): the process-wide ordering of persistent launches keeps
    both on the persistent path, each with its solo ids, pipelined steps
    included."""
    import threading
    shape = synth.GEMMA3_270M.with_ctx(1024).gemma3_mode()
    models = [synth.make_model(shape, seed=31), synth.make_model(shape, seed=32)]
    prompts = [synth.prompt_ids(37, seed=3, vocab=shape.vocab), synth.prompt_ids(52, seed=4, vocab=shape.vocab)]

    def run(e, prompt, out):
        e.prefill(prompt, 0)
        ids = [e.select()]
        for k in range(6):
            ids.append(e.step(ids[-1], len(prompt) + k))
        e.step_submit(ids[-1], len(prompt) + 6)
        for k in range(7, 20):
            e.step_submit(-1, len(prompt) + k)
            ids.append(e.step_collect())
        ids.append(e.step_collect())
        out.append(ids)

    want = []
    for t, p in zip(models, prompts):
        e = engine(shape, t, prefill_batch=32)
        out = []
        run(e, p, out)
        e.close()
        want.append(out[0])
    engines = [engine(shape, t, prefill_batch=32) for t in models]
    outs = [[], []]
    threads = [threading.Thread(target=run, args=(engines[i], prompts[i], outs[i])) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads)
    assert [e.decode_path() for e in engines] == ["fused", "fused"]
    assert outs[0] == [want[0]] and outs[1] == [want[1]]
    for e in engines:
        e.close()
