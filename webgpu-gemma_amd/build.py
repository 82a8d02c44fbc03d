"""Build recipe for libgg.so (gfx950) and the Node-API binding of the JavaScript host.

Called by __graft_entry__.build(); compiles every time it is called.
"""
from __future__ import annotations

import os
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: hipcc must not form v_pk_{add,mul,fma}_f32 from scalar code.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
SOURCES = ["gg_kernels.hip", "gg_decode.hip", "gg_runtime.hip"]
# Per-source options: the persistent decode kernel is one long latency chain
# at one wave per SIMD. Per step, on two boxes each:
# - MFMA results in ordinary VGPRs rather than accumulation registers
#   (-amdgpu-mfma-vgpr-form): 1.4% faster; no copies out of the accumulators;
# - the iterative max-occupancy scheduler at -O2: 0.6% faster than iterative
#   ILP, itself 1.0% faster than the default at -O3 (max-ilp +1.2%,
#   max-memory-clause +4.4%, iterative-minreg +15%; -O1 +5%).
# The later -O2 overrides HIP_FLAGS' -O3.
EXTRA = {"gg_decode.hip": ["-O2", "-mllvm", "-amdgpu-sched-strategy=iterative-maxocc",
                           "-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    return r.stdout


def build_lib() -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    out = os.path.join(LIBDIR, "libgg.so")
    tmp = out + ".tmp"
    objs = []
    for s in SOURCES:
        o = os.path.join(LIBDIR, s.replace(".hip", ".o"))
        _run([HIPCC, *HIP_FLAGS, *EXTRA.get(s, []), "-I", os.path.join(ROOT, "include"), "-c", os.path.join(CSRC, s),
              "-o", o])
        objs.append(o)
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    for o in objs:
        os.remove(o)
    return out


NODE_INCLUDE = "/usr/include/node"


def build_napi() -> str:
    """gg_napi.node: the Node-API binding (C, gcc) linked against libgg.so in
    the same directory. Returns the path, or "" when the Node headers are absent."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        return ""
    out = os.path.join(LIBDIR, "gg_napi.node")
    tmp = out + ".tmp"
    _run(["gcc", "-shared", "-fPIC", "-O2", "-std=c11", "-Wall", "-Werror", "-I", NODE_INCLUDE,
          "-I", os.path.join(ROOT, "include"), os.path.join(PKG, "js", "gg_napi.c"), "-o", tmp,
          "-L", LIBDIR, "-lgg", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_lib())
    print(build_napi())
