"""The device sigmoid (common.h, sigmoid; the standalone op, the CALayer
block and the fused conv epilogue): 1 / (1 + 2^(-x log2 e)), the power on
the transcendental unit (v_exp_f32) and one hardware reciprocal (v_rcp_f32),
each specified to 1 ulp. This restates the operation sequence in numpy fp32,
with the power and the reciprocal correctly rounded and then one ulp off
either way, and holds every combination to the exact function in float64:
the approximation's error is pinned by mathematics, inside the bar the
sigmoid op is held to against the CPU path, |d| <= 4e-7 * (1 + |x|),
including the tails where the power overflows (-> 0) or vanishes (-> 1)."""

import numpy as np

LOG2E = np.float32(1.4426950408889634)


def nudge(v, ulps):
    if ulps == 0:
        return v
    return np.nextafter(v, np.float32(np.inf if ulps > 0 else -np.inf)).astype(np.float32)


def sigmoid_f32(x, exp_ulps=0, rcp_ulps=0):
    f32 = np.float32
    with np.errstate(over="ignore", divide="ignore"):
        t = ((-x).astype(f32) * LOG2E).astype(f32)
        e = nudge(np.exp2(t.astype(np.float64)).astype(f32), exp_ulps)
        s = (f32(1) + e).astype(f32)
        r = nudge((1.0 / s.astype(np.float64)).astype(f32), rcp_ulps)
    return r


def test_sigmoid_within_its_bound():
    x = np.linspace(-120, 120, 2_400_001, dtype=np.float64).astype(np.float32)
    with np.errstate(over="ignore"):
        exact = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    worst = 0.0
    for eu in (-1, 0, 1):
        for ru in (-1, 0, 1):
            got = sigmoid_f32(x, eu, ru).astype(np.float64)
            assert np.isfinite(got).all()
            worst = max(worst, float((np.abs(got - exact) / (1 + np.abs(x))).max()))
    print("worst |d| / (1 + |x|) = %.3g" % worst)
    assert worst <= 1.3e-7


def test_sigmoid_tails_and_specials():
    big = np.array([88.0, 100.0, 1e4, 3e38], np.float32)
    assert (sigmoid_f32(big) == 1.0).all()
    # the power overflows past x = -88.7: the reciprocal of infinity
    assert (sigmoid_f32(-big[1:]) == 0.0).all() and 0.0 <= sigmoid_f32(-big[:1])[0] < 1e-38
    assert sigmoid_f32(np.array([0.0], np.float32))[0] == 0.5
    assert np.isnan(sigmoid_f32(np.array([np.nan], np.float32))[0])
