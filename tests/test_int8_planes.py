"""The int8-plane form the persistent decode kernel gives its FFN
activations before the int8 MFMA products (gg_decode.hip split3 /
planes_value): per 32-element block with m = max|x|, S = m / 127,
p0 = rint(x / S), p1 = rint((x / S - p0) 254), p2 = rint(((x / S - p0) 254 -
p1) 254). Checked in float32 arithmetic like the device: every plane stays in
int8 range (a base of 256 would overflow p1 at 128), and S (p0 + p1 / 254 +
p2 / 254^2) is within 2e-7 m of x -- a few float32 ulps relative to
the block maximum, so the MFMA's exact integer sums lose nothing the float
path would keep."""
import numpy as np


def split3(x: np.ndarray):
    x = x.astype(np.float32)
    m = np.float32(np.max(np.abs(x)))
    inv = np.float32(127.0) / m if m > 0 else np.float32(0.0)
    y = (x * inv).astype(np.float32)
    a = np.rint(y).astype(np.float32)
    r = ((y - a) * np.float32(254.0)).astype(np.float32)
    b = np.rint(r).astype(np.float32)
    c = np.rint(((r - b) * np.float32(254.0)).astype(np.float32)).astype(np.float32)
    return m, a, b, c


def value(m, a, b, c):
    s = np.float64(np.float32(m) * np.float32(1.0 / 127.0))
    return s * (a.astype(np.float64) + b / 254.0 + c / 254.0 ** 2)


def test_planes_range_and_error_bound():
    rng = np.random.default_rng(0)
    blocks = [rng.standard_normal(32) * 10 ** rng.uniform(-8, 4) for _ in range(4000)]
    blocks += [np.zeros(32), np.full(32, 3.0), np.full(32, -2.5), np.r_[1e4, np.zeros(31)],
               np.r_[1.0, np.full(31, 1e-9)], np.linspace(-1, 1, 32), rng.uniform(-127, 127, 32)]
    worst = 0.0
    for x in blocks:
        x = x.astype(np.float32)
        m, a, b, c = split3(x)
        for p in (a, b, c):
            assert np.all(np.abs(p) <= 127), (x, p)
        if m == 0:
            assert not np.any(a) and not np.any(b) and not np.any(c)
            continue
        err = np.max(np.abs(value(m, a, b, c) - x.astype(np.float64))) / float(m)
        worst = max(worst, err)
    assert worst <= 2e-7, worst


def test_base_256_would_overflow():
    # the remainder after rint is in [-0.5, 0.5]: times 254 it stays within
    # int8, times 256 it reaches 128 (the reason for the base)
    y = np.float32(0.5)
    assert np.rint(y * np.float32(254.0)) == 127
    assert np.rint(y * np.float32(256.0)) == 128
