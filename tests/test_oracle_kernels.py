"""Pin each oracle kernel (oracle/gemma_oracle.c) against closed forms,
float64 restatements, invariants and hand-computed cases."""
import numpy as np
import pytest

from gemma_amd import gguf, synth
from oracle import oracle as orc


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


# ---- linearQ8 (shaders.ts:92-151) ----------------------------------------

@pytest.mark.parametrize("rows,k", [(1, 32), (7, 64), (64, 1152), (33, 2048 + 64)])
def test_linear_q8_against_float64(rows, k):
    blocks, x = synth.gemv_operands(rows if rows % 1 == 0 else rows, k, seed=rows * 7 + k)
    y = orc.linear_q8(blocks, x, rows)
    W = gguf.dequantize_q8_0_np(blocks, rows * k).astype(np.float64).reshape(rows, k)
    y64 = W @ x.astype(np.float64)
    cond = np.abs(W) @ np.abs(x.astype(np.float64))
    # sequential fp32 sums: |err| <= ~K * 2^-24 * sum|w x|
    assert np.all(np.abs(y - y64) <= (k + 2) * 2.0 ** -24 * cond + 1e-30)


def test_linear_q8_brute_force_tiny():
    # one row, two blocks, exact small integers: y = sum_b d_b * sum_j q_bj x_j
    q = np.zeros((2, 32), np.int8)
    q[0, :4] = [1, -2, 3, -4]
    q[1, 31] = 5
    blocks = gguf.q8_0_blocks(np.array([0.5, 2.0], np.float16), q)
    x = np.arange(64, dtype=np.float32)
    y = orc.linear_q8(blocks, x, 1)
    expect = 0.5 * (0 * 1 + 1 * -2 + 2 * 3 + 3 * -4) + 2.0 * (63 * 5)
    assert y[0] == expect


def test_linear_q8_orientation():
    # rows are outputs, ne0 (K) is the input: a transposed read would change y
    rows, k = 64, 64
    blocks, x = synth.gemv_operands(rows, k, seed=11)
    W = gguf.dequantize_q8_0_np(blocks, rows * k).reshape(rows, k).astype(np.float64)
    y = orc.linear_q8(blocks, x, rows)
    assert rel_err(y, W @ x) < 1e-5
    assert rel_err(y, W.T @ x) > 0.1


# ---- norms (shaders.ts:25-56, 386-418) ------------------------------------

def test_rms_norm_closed_form():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(1152).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(1152)).astype(np.float32)
    y = orc.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    ref = x64 * w / np.sqrt(np.mean(x64 * x64) + 1e-6)
    assert rel_err(y, ref) < 2e-6
    # invariant: with w = 1 the output has unit RMS
    y1 = orc.rms_norm(x, np.ones_like(x), 0.0)
    assert abs(np.sqrt(np.mean(y1.astype(np.float64) ** 2)) - 1) < 1e-6


def test_rms_norm_eps_dominates_zero_input():
    x = np.zeros(640, np.float32)
    y = orc.rms_norm(x, np.ones(640, np.float32), 1e-6)
    assert np.all(y == 0)


def test_fused_norm_add():
    rng = np.random.default_rng(6)
    x, r = rng.standard_normal((2, 640)).astype(np.float32)
    w = (1 + rng.standard_normal(640) * 0.1).astype(np.float32)
    y = orc.fused_norm_add(x, w, r, 1e-6)
    x64 = x.astype(np.float64)
    ref = r + x64 * w / np.sqrt(np.mean(x64 * x64) + 1e-6)
    assert rel_err(y, ref) < 2e-6


# ---- GeGLU (shaders.ts:153-170) -------------------------------------------

def test_gelu_mul_closed_form_and_limits():
    g = np.linspace(-30, 30, 4001).astype(np.float32)
    u = np.full_like(g, 1.5)
    y = orc.gelu_mul(g, u).astype(np.float64)
    g64 = g.astype(np.float64)
    t = np.clip(np.sqrt(2 / np.pi) * g64 * (1 + 0.044715 * g64 ** 2), -15, 15)
    ref = 0.5 * g64 * (1 + np.tanh(t)) * 1.5
    assert np.all(np.abs(y - ref) <= 4e-7 * np.maximum(np.abs(ref), 1.0))
    assert orc.gelu_mul(np.zeros(1), np.ones(1))[0] == 0.0
    # saturated region: tanh(15) rounds to 1 in f32 -> gelu(x) = x
    assert orc.gelu_mul(np.array([20.0]), np.array([2.0]))[0] == 40.0


# ---- per-head norm + RoPE (shaders.ts:420-467) ------------------------------

def test_rope_freq_against_float64():
    for theta in (1e4, 1e6):
        f = np.array([orc.rope_freq(i, 256, theta) for i in range(128)])
        ref = 1.0 / np.power(theta, 2.0 * np.arange(128) / 256)
        assert rel_err(f, ref) < 1e-6
        assert f[0] == 1.0


def _f64_norm_rope(x, w, nh, pos, theta, eps=1e-6):
    x = x.reshape(nh, 256).astype(np.float64)
    x = x * w / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps)
    i = np.arange(128)
    freq = np.array([orc.rope_freq(j, 256, theta) for j in i], dtype=np.float32)
    ang = (np.float32(pos) * freq).astype(np.float64)
    a, b = x[:, :128], x[:, 128:]
    return np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], 1).reshape(-1)


@pytest.mark.parametrize("pos,theta", [(0, 1e6), (1, 1e4), (777, 1e6), (2047, 1e4), (32767, 1e6)])
def test_norm_rope_against_float64(pos, theta):
    rng = np.random.default_rng(pos)
    x = rng.standard_normal(4 * 256).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    y = orc.per_head_norm_rope(x, w, 4, 256, 1e-6, pos, theta)
    assert rel_err(y, _f64_norm_rope(x, w, 4, pos, theta)) < 3e-6


def test_rope_invariants():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(256).astype(np.float32)
    w = np.ones(256, np.float32)
    normed = orc.per_head_norm_rope(x, w, 1, 256, 1e-6, 0, 1e6)   # pos 0: rotation is the identity
    ref = orc.rms_norm(x, w, 1e-6)
    assert np.array_equal(normed, ref)
    y = orc.per_head_norm_rope(x, w, 1, 256, 1e-6, 321, 1e4)
    pair_norm = lambda v: v[:128] ** 2 + v[128:] ** 2  # noqa: E731
    assert np.allclose(pair_norm(y.astype(np.float64)), pair_norm(ref.astype(np.float64)), rtol=1e-5)


# ---- attention (shaders.ts:229-325) -------------------------------------

def test_attention_single_position_returns_v():
    rng = np.random.default_rng(10)
    q = rng.standard_normal(4 * 256).astype(np.float32)
    kc = rng.standard_normal((8, 256)).astype(np.float32)
    vc = rng.standard_normal((8, 256)).astype(np.float32)
    out, sc = orc.attention(q, kc, vc, 4, 1, 256, 5, 5, 0.0625)
    assert np.all(sc == 1.0)
    assert np.array_equal(out.reshape(4, 256), np.tile(vc[5], (4, 1)))


def test_attention_against_float64_and_window():
    rng = np.random.default_rng(11)
    q = rng.standard_normal(4 * 256).astype(np.float32)
    kc = rng.standard_normal((600, 256)).astype(np.float32)
    vc = rng.standard_normal((600, 256)).astype(np.float32)
    for lo, hi in [(0, 599), (88, 599), (0, 0), (300, 310)]:
        out, _ = orc.attention(q, kc, vc, 4, 1, 256, lo, hi, 0.0625)
        s = q.reshape(4, 256).astype(np.float64) @ kc[lo:hi + 1].T.astype(np.float64) * 0.0625
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        ref = (p @ vc[lo:hi + 1].astype(np.float64)).reshape(-1)
        assert rel_err(out, ref) < 1e-5


def test_attention_uniform_scores_average_v():
    rng = np.random.default_rng(12)
    kc = rng.standard_normal((16, 256)).astype(np.float32)
    vc = rng.standard_normal((16, 256)).astype(np.float32)
    out, _ = orc.attention(np.zeros(4 * 256, np.float32), kc, vc, 4, 1, 256, 0, 15, 0.0625)
    assert rel_err(out.reshape(4, 256)[2], vc.astype(np.float64).mean(0)) < 1e-6


# ---- argmax / topk256 (shaders.ts:327-384) --------------------------------

def brev8(c):
    return int(f"{c:08b}"[::-1], 2)


def closed_form_argmax(v):
    """Winner of the reference reduction: the largest value above -1e30; among
    equal maxima the smallest 8-bit bit-reversed stride class, then the
    smallest index; index 0 when nothing exceeds -1e30."""
    v = np.asarray(v, np.float32)
    ok = ~np.isnan(v) & (v > np.float32(-1e30))
    if not ok.any():
        return 0
    m = v[ok].max()
    idx = np.nonzero(ok & (v == m))[0]
    return int(min(idx, key=lambda i: (brev8(i % 256), i)))


@pytest.mark.parametrize("seed", range(6))
def test_argmax_tie_rule(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 5000))
    v = rng.integers(-3, 3, size=n).astype(np.float32)   # many exact ties
    if seed % 2:
        v[rng.integers(0, n, size=max(1, n // 10))] = np.nan
    assert orc.argmax(v) == closed_form_argmax(v)


def test_argmax_edge_cases():
    assert orc.argmax(np.full(300, -np.inf, np.float32)) == 0
    assert orc.argmax(np.full(300, -1e30, np.float32)) == 0
    assert orc.argmax(np.full(300, np.nan, np.float32)) == 0
    v = np.zeros(512, np.float32)
    v[[1, 128, 256 + 64]] = 5.0   # classes 1 (brev 128), 128 (brev 1), 64 (brev 2)
    assert orc.argmax(v) == 128
    v = np.zeros(1024, np.float32)
    v[[3, 259, 515]] = 1.0        # same class 3: first occurrence
    assert orc.argmax(v) == 3
    v = np.zeros(10, np.float32)
    v[7] = np.inf
    assert orc.argmax(v) == 7


def test_topk256_is_per_class_first_max():
    rng = np.random.default_rng(21)
    v = rng.integers(0, 4, size=262144).astype(np.float32)
    vals, ids = orc.topk256(v)
    cls = v.reshape(-1, 256)
    assert np.array_equal(vals, cls.max(0))
    first = np.argmax(cls == cls.max(0), axis=0) * 256 + np.arange(256)
    assert np.array_equal(ids, first)
    # short vocab: classes without any element report (-1e30, 0)
    vals, ids = orc.topk256(np.ones(100, np.float32))
    assert np.all(vals[100:] == np.float32(-1e30)) and np.all(ids[100:] == 0)


# ---- host sampler (engine.ts:862-901) -------------------------------------

def _cands(vals, ids=None):
    v = np.full(256, -1e30, np.float32)
    v[:len(vals)] = vals
    i = np.arange(256, dtype=np.uint32) if ids is None else np.asarray(ids, np.uint32)
    return v, i


def test_sampler_greedy_and_stable_ties():
    v, i = _cands([1.0, 3.0, 3.0, 2.0])
    assert orc.sample_candidates(v, i, [], 0.0, 0.9, 1.0, 0.5) == 1   # stable: first of the tie
    i2 = i.copy()
    i2[1], i2[2] = 9000, 17
    assert orc.sample_candidates(v, i2, [], 0.0, 0.9, 1.0, 0.5) == 9000


def test_sampler_repetition_penalty():
    v, i = _cands([2.0, 1.9, -1.0, -1.1])
    # seen id 0: 2.0 / 1.2 = 1.667 < 1.9 -> id 1 wins at T=0
    assert orc.sample_candidates(v, i, [0], 0.0, 0.9, 1.2, 0.0) == 1
    # penalty <= 1 or empty set: untouched
    assert orc.sample_candidates(v, i, [0], 0.0, 0.9, 1.0, 0.0) == 0
    assert orc.sample_candidates(v, i, [], 0.0, 0.9, 1.2, 0.0) == 0
    # negative logits are multiplied: -1.0 * 1.2 = -1.2 < -1.1
    v2, i2 = _cands([-1.0, -1.1])
    assert orc.sample_candidates(v2, i2, [0], 0.0, 0.9, 1.2, 0.0) == 1


def test_sampler_top_p_walk():
    # probs (T=1): 1, 0.5, 0.25, then ~0; sum 1.75; cumulative 0.571, 0.857, 1.0
    v, i = _cands([0.0, np.log(0.5), np.log(0.25)], ids=np.arange(256) + 1000)
    s = lambda u, p=0.9: orc.sample_candidates(v, i, [], 1.0, p, 1.0, u)  # noqa: E731
    assert s(0.50) == 1000   # r = 0.875 -> first subtraction reaches <= 0
    assert s(0.60) == 1001   # r = 1.05
    assert s(0.99) == 1002   # r = 1.7325
    assert s(0.99, p=0.5) == 1000   # cutoff 1
    assert s(0.99, p=0.8) == 1001   # cutoff 2 (0.857 >= 0.8)
    assert s(0.0) == 1000    # r = 0 -> r - p0 <= 0


def test_sampler_temperature_sharpens():
    v, i = _cands([1.0, 0.0])
    # T = 0.1: p1 = exp(-10) ~ 4.5e-5 relative; u = 0.9999 still lands on id 0
    assert orc.sample_candidates(v, i, [], 0.1, 1.0, 1.0, 0.9999) == 0
    # T = 10: p1 = exp(-0.1) = 0.905, sum 1.905; u = 0.9 -> r = 1.714 -> id 1
    assert orc.sample_candidates(v, i, [], 10.0, 1.0, 1.0, 0.9) == 1
