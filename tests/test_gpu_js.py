"""The JavaScript host on the GPU through the Node-API binding: two generate()
turns (greedy, then sampled with a seeded draw) on a tiny GGUF written by
gemma_amd.gguf. On the persistent kernel's path generate() keeps one step
queued ahead (stepSubmit / stepCollect, each step taking the previous id on
the device); every collected step is logged with its input id resolved. On
the graph path (GG_DECODE=graph) it awaits each step. The binding calls the
host made are replayed through the Python C-ABI binding as sequential steps
and must give the same ids (a step queued past a turn's end included); the
greedy turn must also match the oracle."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from gemma_amd import capi, synth
from oracle import oracle as orc

from gpu_util import say

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
NODE = shutil.which("node")


@pytest.mark.skipif(NODE is None, reason="node is not installed")
@pytest.mark.parametrize("attention,path", [("reference", "fused"), ("gemma3", "fused"), ("gemma3", "graph")])
def test_js_host_on_gpu(gpu, tmp_path, attention, path):
    say("js host", attention, path)
    shape = synth.TINY.with_ctx(256)
    tensors = synth.make_model(shape, seed=9)
    g = str(tmp_path / "tiny.gguf")
    synth.write_model_gguf(g, shape, tensors=tensors)
    env = dict(os.environ)
    if path == "graph":
        env["GG_DECODE"] = "graph"   # the binding then reports decodePath 0
    r = subprocess.run([NODE, os.path.join(HERE, "js", "gpu_generate.js"), g, attention], stdout=subprocess.PIPE,
                       stderr=subprocess.PIPE, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    log = out["log"]
    # generate() queues steps only on the persistent kernel's path; on the
    # graph path a queued submit would block the event loop
    queued = [c for c in log if c.get("queued")]
    assert (len(queued) > 0) == (path == "fused"), path
    run_shape = shape.gemma3_mode(window=512) if attention == "gemma3" else shape.reference_mode()

    # replay the same calls through the Python binding of the C-ABI
    # the host's default: the batched MFMA prefill, the whole prompt per slice
    e = capi.Engine(run_shape.gg_config(prefill_batch=min(4096, run_shape.ctx)))
    e.upload_model(tensors)
    e.finalize()
    for c in log:
        if c["op"] == "prefill":
            e.prefill(np.array(c["ids"], np.int32), c["pos"])
        elif c["op"] == "penaltyReset":
            e.penalty_reset()
        elif c["op"] == "penaltyAdd":
            e.penalty_add(c["ids"])
        elif c["op"] == "select":
            assert e.select(c["t"], c["p"], c["r"], c["u"]) == c["id"]
        else:
            assert e.step(c["tok"], c["pos"], c["t"], c["p"], c["r"], c["u"]) == c["id"]
    e.close()

    # the greedy first turn against the oracle
    o = orc.OracleModel(run_shape, tensors)
    first = log[[c["op"] for c in log].index("prefill")]
    o.prefill(np.array(first["ids"], np.int32), 0)
    sel = [c for c in log if c["op"] in ("select", "step") and c["t"] == 0]
    seen = list(first["ids"])           # the turn's penalty set: its prompt + the selected ids
    assert sel[0]["op"] == "select"
    assert o.select(0.0, sel[0]["p"], sel[0]["r"], 0.0, seen=seen) == sel[0]["id"]
    seen.append(sel[0]["id"])
    for c in sel[1:]:
        o.forward(c["tok"], c["pos"])
        assert o.select(0.0, c["p"], c["r"], 0.0, seen=seen) == c["id"]
        seen.append(c["id"])
    o.close()
    # positions: the second turn's prefill starts where the first turn's KV ends
    pf = [c for c in log if c["op"] == "prefill"]
    greedy_writes = sum(1 for c in sel if c["op"] == "step" and not c.get("dropped"))
    assert pf[1]["pos"] == len(pf[0]["ids"]) + greedy_writes
    assert pf[1]["ids"][0] != 2        # the turn suffix has no BOS
