"""Context lifetime of the Node-API binding (webgpu-gemma_amd/js/gg_napi.c)
on the CPU: the binding is compiled against a stub libgg (tests/js/stub_gg.c)
whose prefill/select/step sleep, once plainly and once with AddressSanitizer
on the binding and the stub, and tests/js/napi_lifecycle.js starts a second
job on a busy context, destroys a context during a step, calls a destroyed
context and drops a handle to the garbage collector during a step. The stub
aborts on any use after gg_destroy or overlapping calls; the test also checks
from the stub's event log that each context is destroyed once, after its last
call ended."""
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
NODE = shutil.which("node")
NODE_INCLUDE = "/usr/include/node"


def build(tmp, asan):
    san = ["-fsanitize=address", "-fno-omit-frame-pointer"] if asan else []
    common = ["gcc", "-shared", "-fPIC", "-O1", "-g", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include")]
    subprocess.run(common + san + [os.path.join(HERE, "js", "stub_gg.c"), "-o", os.path.join(tmp, "libgg.so")],
                   check=True)
    subprocess.run(common + san + ["-I", NODE_INCLUDE, os.path.join(ROOT, "webgpu-gemma_amd", "js", "gg_napi.c"),
                                   "-o", os.path.join(tmp, "gg_napi.node"), "-L", tmp, "-lgg",
                                   "-Wl,-rpath," + tmp], check=True)


def check_log(stderr):
    assert "USE AFTER DESTROY" not in stderr and "CONCURRENT CALL" not in stderr, stderr
    events = re.findall(r"^stub: (\S+) (\d+)$", stderr, re.M)
    per = {}
    for ev, cid in events:
        per.setdefault(cid, []).append(ev)
    # context 1: finalize, two steps, destroyed once after the second step ended
    assert per["1"] == ["create", "finalize", "finalize-end", "step", "step-end", "step", "step-end", "destroy"], per
    # context 2: destroyed after its prefill ended
    assert per["2"] == ["create", "prefill", "prefill-end", "destroy"], per
    # context 3: a step; if the collector finalized the handle, destroy comes after the step
    assert per["3"][:3] == ["create", "step", "step-end"] and per["3"][3:] in ([], ["destroy"]), per
    # context 4: pipelined steps, destroyed after the second collect ended
    assert per["4"] == ["create", "step_submit", "step_submit-end", "step_collect", "step_collect-end",
                        "step_submit", "step_submit-end", "step_collect", "step_collect-end", "destroy"], per


@pytest.mark.skipif(NODE is None or not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")),
                    reason="node or its headers are not installed")
@pytest.mark.parametrize("asan", [False, True], ids=["plain", "asan"])
def test_napi_context_lifetime(tmp_path, asan):
    build(str(tmp_path), asan)
    env = dict(os.environ)
    if asan:
        lib = subprocess.run(["gcc", "-print-file-name=libasan.so"], stdout=subprocess.PIPE, text=True,
                             check=True).stdout.strip()
        env["LD_PRELOAD"] = lib
        env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    r = subprocess.run([NODE, "--expose-gc", os.path.join(HERE, "js", "napi_lifecycle.js"), str(tmp_path)],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=60, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.splitlines()[-1] == "lifecycle passed", r.stdout + r.stderr
    assert "AddressSanitizer" not in r.stderr, r.stderr
    check_log(r.stderr)
