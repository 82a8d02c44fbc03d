"""Single-kernel parity on the GPU through the C-ABI kernel entry points:
Q8_0 dequant (bit-exact), Q8_0 GEMV at the Gemma-3-1B shapes (1e-4 relative),
and the vocab selector (argmax tie rule, topk256, sampler) on identical logits."""
import numpy as np
import pytest

from gemma_amd import capi, gguf, synth
from oracle import oracle as orc

from gpu_util import dev, empty, host, rel, say, stream

pytestmark = pytest.mark.gpu

GEMV_SHAPES = [(1152, 1536), (1024, 1152), (1152, 13824), (6912, 1152), (1152, 262144)]


def test_dequant_bit_exact(gpu):
    rng = np.random.default_rng(0)
    nb = 1 << 16
    q = rng.integers(-128, 128, size=(nb, 32)).astype(np.int8)
    codes = rng.integers(0, 65536, size=nb).astype(np.uint16)
    codes[:64] = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x3C00] + \
        list(range(0x0002, 0x0002 + 53))
    blocks = gguf.q8_0_blocks(codes.view(np.float16), q)
    say("dequant", nb * 32)
    src = dev(blocks)
    out = empty(nb * 32 * 4)
    capi.q8_0_dequant(src.data_ptr(), out.data_ptr(), nb * 32, stream())
    got = host(out, np.float32)
    ref = orc.q8_0_dequant(blocks, nb * 32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("k,n", GEMV_SHAPES + [(640, 1536), (2048, 640), (8192, 64), (64, 64)])
def test_q8_0_gemv_shapes(gpu, k, n):
    say("gemv", k, n)
    blocks, x = synth.gemv_operands(n, k, seed=k + n)
    src = dev(blocks)
    w = empty(capi.q8_0_packed_size(n, k))
    capi.q8_0_repack(src.data_ptr(), w.data_ptr(), n, k, stream())
    xd = dev(x)
    y = empty(n * 4)
    capi.q8_0_gemv(w.data_ptr(), xd.data_ptr(), y.data_ptr(), n, k, stream())
    got = host(y, np.float32)
    ref = orc.linear_q8(blocks, x, n)
    assert rel(got, ref) < 1e-4
    # and every row within the fp32 summation bound of the exact product
    W = gguf.dequantize_q8_0_np(blocks, n * k).reshape(n, k)
    if n <= 16384:
        y64 = W.astype(np.float64) @ x.astype(np.float64)
        cond = np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64))
        assert np.all(np.abs(got - y64) <= (k + 2) * 2.0 ** -24 * cond)


@pytest.mark.parametrize("k,n", [(1152, 1536), (1152, 262144 // 16), (6912, 1152)])
def test_gemv_repack_preserves_bytes(gpu, k, n):
    blocks, _ = synth.gemv_operands(n, k, seed=5)
    src = dev(blocks)
    w = empty(capi.q8_0_packed_size(n, k))
    capi.q8_0_repack(src.data_ptr(), w.data_ptr(), n, k, stream())
    packed = host(w, np.uint8)
    # item-planar layout: pair (row r, col c) is slot (c % CI) * GR + r % GR of
    # item (r // GR) * KpS + c // CI (4352 bytes each); dword j of slot s sits
    # at 1024 (j // 4) + 16 s + 4 (j % 4) for j < 16 and at 4096 + 4 s for j = 16
    kp = k // 64
    gr = 64 if n >= 8192 else 8
    ci = 64 // gr
    kps = -(-kp // ci)
    assert packed.nbytes == n // gr * kps * 4352
    pairs = blocks.reshape(n, kp, 68)
    rng = np.random.default_rng(0)

    def pair_at(r, c):
        item = (r // gr * kps + c // ci) * 4352
        slot = (c % ci) * gr + r % gr
        offs = [item + (1024 * (j // 4) + 16 * slot + 4 * (j % 4) if j < 16 else 4096 + 4 * slot) for j in range(17)]
        return np.concatenate([packed[o:o + 4] for o in offs])

    for r, c in [(0, 0), (63, kp - 1), (64, 0), (n - 1, kp - 1)] + [(int(a), int(b)) for a, b in
                                                                    zip(rng.integers(0, n, 50), rng.integers(0, kp, 50))]:
        assert np.array_equal(pair_at(r, c), pairs[r, c])
    # every GGUF byte appears exactly once: total of all pairs equals the input bytes
    used = n * kp * 68
    assert used == blocks.nbytes


def _select(logits, seen_ids, T, p, rep, u, want_topk=True):
    n = logits.size
    ld = dev(logits.astype(np.float32))
    ws = empty(capi.select_workspace_size(n))
    topk = empty(512 * 4)
    seen = None
    if len(seen_ids):
        bm = np.zeros((n + 31) // 32, np.uint32)
        for t in seen_ids:
            bm[t >> 5] |= np.uint32(1 << (t & 31))
        seen = dev(bm)
    tok = capi.select_logits(ld.data_ptr(), n, seen.data_ptr() if seen is not None else None, T, p, rep, u,
                             ws.data_ptr(), topk.data_ptr(), stream())
    raw = host(topk, np.uint32)
    return tok, raw[0::2].view(np.float32), raw[1::2]


@pytest.mark.parametrize("seed", range(4))
def test_argmax_tie_rule_on_gpu(gpu, seed):
    rng = np.random.default_rng(seed)
    n = [262144, 2048, 1000, 256 * 37][seed]
    v = rng.integers(-2, 3, size=n).astype(np.float32)   # heavy ties
    if seed == 1:
        v[rng.integers(0, n, 50)] = np.nan
    tok, vals, ids = _select(v, [], 0.0, 0.9, 1.0, 0.0)
    assert tok == orc.argmax(v)
    rv, ri = orc.topk256(v)
    assert np.array_equal(vals, rv) and np.array_equal(ids, ri)


def test_argmax_all_below_floor(gpu):
    v = np.full(4096, -np.inf, np.float32)
    tok, vals, ids = _select(v, [], 0.0, 0.9, 1.0, 0.0)
    assert tok == 0 and np.all(vals == np.float32(-1e30)) and np.all(ids == 0)


@pytest.mark.parametrize("seed", range(8))
def test_sampler_matches_host_semantics(gpu, seed):
    rng = np.random.default_rng(100 + seed)
    n = 262144
    v = (rng.standard_normal(n) * 2).astype(np.float32)
    seen = list(rng.integers(0, n, size=200))
    vals, ids = orc.topk256(v)
    # make some candidates seen
    seen += [int(i) for i in ids[rng.integers(0, 256, 20)]]
    for T, p, rep in [(0.7, 0.9, 1.2), (1.0, 0.5, 1.0), (0.0, 0.9, 1.2), (1.3, 0.99, 1.5)]:
        u = float(rng.random())
        tok, _, _ = _select(v, seen, T, p, rep, u)
        assert tok == orc.sample_candidates(vals, ids, seen, T, p, rep, u), (T, p, rep, u)
    # the ends of the walk and of the top-p cutoff: draws at 0 and just below
    # 1, top-p 1 (the cumulative sum may never reach it: all 256 candidates),
    # a top-p below the first probability (one candidate), and a near-flat
    # distribution at a high temperature (the longest walks)
    for T, p, rep, u in [(0.7, 0.9, 1.0, 0.0), (0.7, 0.9, 1.0, 1.0 - 2.0 ** -40), (0.7, 1.0, 1.2, float(rng.random())),
                         (0.7, 1.0, 1.0, 1.0 - 2.0 ** -40), (0.7, 1e-6, 1.0, float(rng.random())),
                         (50.0, 0.999, 1.0, float(rng.random())), (50.0, 1.0, 1.0, 1.0 - 2.0 ** -40)]:
        tok, _, _ = _select(v, seen, T, p, rep, u)
        assert tok == orc.sample_candidates(vals, ids, seen, T, p, rep, u), (T, p, rep, u)
