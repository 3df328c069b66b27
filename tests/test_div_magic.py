"""The block maps' divisions as multiplies (exec_hip.cpp div_magic, used by
pointwise.h mdiv): n / d == umulhi(2 n, m) >> s for every n < 2^31, with
s = ceil(log2 d), m = ceil(2^(31 + s) / d). Checked exhaustively where n is
small and at every multiple of d (and its neighbours) near the ends of the
range, for the divisors the MAXIM maps use and for the extremes of d."""
import numpy as np
import pytest


def magic(d):
    s = 0
    while (1 << s) < d:
        s += 1
    m = ((1 << (31 + s)) + d - 1) // d
    assert m < 1 << 32
    return m, s


def mdiv(n, m, s):
    n = np.asarray(n, dtype=np.uint64)
    return ((2 * n * np.uint64(m)) >> np.uint64(32)) >> np.uint64(s)


@pytest.mark.parametrize("d", [1, 2, 3, 4, 7, 8, 10, 14, 16, 20, 28, 40, 64, 70, 256, 280, 1120, 4480,
                               17920, 71680, 286720, 4096 * 4096, (1 << 31) - 1])
def test_division_by_multiply(d):
    m, s = magic(d)
    n = np.arange(0, 1 << 20, dtype=np.uint64)
    assert np.array_equal(mdiv(n, m, s), n // np.uint64(d))
    top = np.uint64((1 << 31) - 1)
    hi = top - np.arange(0, 1 << 16, dtype=np.uint64)
    assert np.array_equal(mdiv(hi, m, s), hi // np.uint64(d))
    k = np.arange(max(1, ((1 << 31) - (1 << 18)) // d), (1 << 31) // d + 1, dtype=np.uint64)
    for delta in (0, 1):
        q = k * np.uint64(d) - np.uint64(delta)
        q = q[q <= top]
        assert np.array_equal(mdiv(q, m, s), q // np.uint64(d))
