"""gg_select_logits_noalloc (the selector on the library's static per-device
workspace) against gg_select_logits (the same kernels on a caller-provided
workspace): identical token and topk256 on two calls in a row, the second
over a smaller vocabulary, for argmax and for the sampler with a penalty
bitmap; the oracle's argmax / topk256 pin the greedy case."""
import numpy as np
import pytest

from gemma_amd import capi
from oracle import oracle as orc

from gpu_util import dev, empty, host, say, stream

pytestmark = pytest.mark.gpu


def _bitmap(n, ids):
    bm = np.zeros((n + 31) // 32, np.uint32)
    for t in ids:
        bm[t >> 5] |= np.uint32(1 << (int(t) & 31))
    return dev(bm)


def _both(logits, seen_ids, T, p, rep, u):
    n = logits.size
    ld = dev(logits.astype(np.float32))
    seen = _bitmap(n, seen_ids) if len(seen_ids) else None
    sp = seen.data_ptr() if seen is not None else None
    ws = empty(capi.select_workspace_size(n))
    top_a = empty(512 * 4)
    top_b = empty(512 * 4)
    tok_a = capi.select_logits(ld.data_ptr(), n, sp, T, p, rep, u, ws.data_ptr(), top_a.data_ptr(), stream())
    tok_b = capi.select_logits_noalloc(ld.data_ptr(), n, sp, T, p, rep, u, top_b.data_ptr(), stream())
    return tok_a, host(top_a, np.uint32), tok_b, host(top_b, np.uint32)


@pytest.mark.parametrize("mode", ["argmax", "sampler"])
def test_noalloc_select_matches_workspace_entry(gpu, mode):
    rng = np.random.default_rng(7 if mode == "argmax" else 8)
    for n in (262144, 1000):   # second call smaller: stale scratch from the first must not leak in
        say("noalloc select", mode, n)
        if mode == "argmax":
            v = rng.integers(-3, 4, size=n).astype(np.float32)   # ties
            tok_a, ta, tok_b, tb = _both(v, [], 0.0, 0.9, 1.0, 0.0)
            assert tok_a == tok_b == orc.argmax(v)
            rv, ri = orc.topk256(v)
            assert np.array_equal(tb[0::2].view(np.float32), rv) and np.array_equal(tb[1::2], ri)
        else:
            v = (rng.standard_normal(n) * 2).astype(np.float32)
            seen = rng.integers(0, n, size=64)
            tok_a, ta, tok_b, tb = _both(v, seen, 0.8, 0.9, 1.3, float(rng.random()))
            assert tok_a == tok_b and 0 <= tok_b < n
        assert np.array_equal(ta, tb)


def test_noalloc_select_without_topk_output(gpu):
    rng = np.random.default_rng(9)
    for n in (4096, 300):
        v = rng.standard_normal(n).astype(np.float32)
        ld = dev(v)
        tok = capi.select_logits_noalloc(ld.data_ptr(), n, None, 0.0, 0.9, 1.0, 0.0, None, stream())
        assert tok == orc.argmax(v)
