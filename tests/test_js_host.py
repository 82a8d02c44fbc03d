"""The JavaScript host (webgpu-gemma_amd/js) on the CPU: Node runs
tests/js/host_tests.js -- tokenizer and chat template (tokenizer.ts,
conversation.ts), the GGUF reader on a file written by gemma_amd.gguf, and
generate()'s turn logic (engine.ts:957-1031) against a recording fake of the
Node-API binding."""
import hashlib
import json
import os
import shutil
import subprocess
from dataclasses import replace

import numpy as np
import pytest

from gemma_amd import gguf, synth

HERE = os.path.dirname(os.path.abspath(__file__))
NODE = shutil.which("node")


def write_tiny(path):
    # rope bases other than the 1e6 / 1e4 defaults, so the test sees the file's values reach create()
    shape = replace(synth.TINY, theta_global=5e5)
    tensors = synth.make_model(shape, seed=3)
    synth.write_model_gguf(path, shape, tensors=tensors, rope_base_swa=2e4)
    r = gguf.GGUFFile(path)
    exp = {"data_offset": r.data_offset, "hidden": shape.hidden, "layers": shape.layers, "inter": shape.inter,
           "vocab": shape.vocab, "file_ctx": max(shape.ctx, 32768), "rope_base": 5e5, "rope_base_swa": 2e4,
           "tensors": []}
    for t in r.tensors:
        b = np.ascontiguousarray(tensors[t.name][2]).tobytes()
        assert bytes(r.tensor_bytes(t)) == b
        exp["tensors"].append({"name": t.name, "dims": [int(d) for d in t.dims], "type": int(t.ggml_type),
                               "offset": int(t.offset), "nbytes": len(b), "sha256": hashlib.sha256(b).hexdigest()})
    return exp


@pytest.mark.skipif(NODE is None, reason="node is not installed")
def test_js_host(tmp_path):
    g = str(tmp_path / "tiny.gguf")
    exp = write_tiny(g)
    ej = str(tmp_path / "expect.json")
    with open(ej, "w") as f:
        json.dump(exp, f)
    r = subprocess.run([NODE, os.path.join(HERE, "js", "host_tests.js"), g, ej], stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    assert "passed" in r.stdout.splitlines()[-1], r.stdout
