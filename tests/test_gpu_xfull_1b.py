"""Gemma-3-1B at full size, greedy decode after a 2048-token context: a 2048-token seeded prompt,
then 256 greedy tokens at batch 1, against the oracle run independently over
the same 2048 positions (engine.ts:735-802 per token, 904-915 per step).
The GPU fills its cache with the batched MFMA prefill and decodes on the
persistent kernel; the oracle runs the reference's token-by-token pass.
Checked: every K/V row of layers 0, 5, 11 and 25 after the prompt (RoPE
rows far past the first 256 positions), every greedy id, and the per-layer
hidden states and logits within 1e-3 at every 32nd step. About two minutes
of oracle time on 16 host cores."""
import time

import numpy as np
import pytest

from gemma_amd import capi, synth
from oracle import oracle as orc

from gpu_util import rel, say

pytestmark = pytest.mark.gpu

TOL = 1e-3


def test_1b_config3_prefill_2048_then_256_greedy(gpu):
    shape = synth.GEMMA3_1B.with_ctx(4096).gemma3_mode()
    say("config3: build model")
    t = synth.make_model(shape, seed=1)
    prompt = synth.prompt_ids(2048, seed=2048, vocab=shape.vocab)
    e = capi.Engine(shape.gg_config(prefill_batch=2048))
    e.upload_model(t)
    e.finalize()
    assert e.decode_path() == "fused"
    e.prefill(prompt, 0)
    tok = e.select()
    o = orc.OracleModel(shape, t)
    t0 = time.time()
    for i in range(0, 2048, 256):
        o.prefill(prompt[i:i + 256], i)
        say(f"config3: oracle prefill {i + 256}/2048 ({time.time() - t0:.0f} s)")
    for l in (0, 5, 11, 25):
        kg = e.read(capi.READ_K_CACHE, l).reshape(shape.ctx, 256)[:2048]
        vg = e.read(capi.READ_V_CACHE, l).reshape(shape.ctx, 256)[:2048]
        kr = o.buffer(orc.GOR_K_CACHE, l).reshape(shape.ctx, 256)[:2048]
        vr = o.buffer(orc.GOR_V_CACHE, l).reshape(shape.ctx, 256)[:2048]
        for p0 in range(0, 2048, 256):   # per block of rows: no large row hides a small one
            assert rel(kg[p0:p0 + 256], kr[p0:p0 + 256]) < TOL, f"layer {l} K rows {p0}.."
            assert rel(vg[p0:p0 + 256], vr[p0:p0 + 256]) < TOL, f"layer {l} V rows {p0}.."
    ref = o.select()
    assert tok == ref, "first token after the prompt"
    pos = 2048
    for step in range(255):
        nxt = e.step(tok, pos)
        o.forward(tok, pos)
        ref = o.select()
        if step % 32 == 0:
            say(f"config3: step {step} ({time.time() - t0:.0f} s)")
            for l in range(shape.layers):
                r = rel(e.read(capi.READ_LAYER_HIDDEN, l), o.buffer(orc.GOR_LAYER_HIDDEN, l))
                assert r < TOL, f"step {step} layer {l} hidden {r:.2e}"
            assert rel(e.read(capi.READ_LOGITS), o.buffer(orc.GOR_LOGITS)) < TOL
        assert nxt == ref, f"token {step + 2} of 256 differs"
        tok, pos = nxt, pos + 1
    o.close()
    e.close()
