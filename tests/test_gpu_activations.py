"""The device GELU and sigmoid (common.h: a fitted exponent polynomial and a
hardware exp2 for Phi, a hardware exp2 and reciprocal for the sigmoid) as
standalone ops on the values where their approximations have edges - the
GELU's clamp at |x| = 6, the exponent's overflow and underflow, signed
zeros, denormals, the largest floats and NaN - against the CPU path (libm
erff and expf) at the activation bar, |d| <= 4e-7 * (1 + |x|): NaN exactly
where the CPU path gives NaN, nothing else non-finite."""

import numpy as np
import pytest

from test_gpu_pointwise import oracle_plan, run_plan

pytestmark = pytest.mark.gpu

EDGES = [0.0, -0.0, 1e-30, -1e-30, 1e-45, -1e-45, 5.999, -5.999, 6.0, -6.0, 6.001, -6.001, 10.0, -10.0,
         30.0, -30.0, 88.7, -88.7, 89.0, -89.0, 100.0, -100.0, 1e4, -1e4, 1e30, -1e30, 3.4e38, -3.4e38,
         float("nan")]


@pytest.mark.parametrize("kind", ["gelu", "sigmoid"])
def test_activation_edges_against_the_cpu_path(gpu_ok, kind):
    from maxim_amd import plan as P
    x = np.concatenate([np.linspace(-12, 12, 24001), EDGES, [0.5, 0.25]]).astype(np.float32)
    n = x.size
    assert n % 4 == 0
    op = P.GELU if kind == "gelu" else P.SIGMOID
    bufs = [(1, 1, n), (1, 1, n)]
    cp = P.CustomPlan(bufs, [P.make_op(op, dst=1, src=0, n=n)], [], input=0, output=1, align=1)
    got, steps = run_plan(cp, {0: x.reshape(1, 1, n)}, 1)
    want = oracle_plan(cp, {0: x.reshape(1, 1, n)}, 1)
    got, want = got.ravel(), want.ravel()
    print(kind, "kernels", [k for _, _, k in steps])
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all(), x[np.isnan(got) != nan]
    assert np.isfinite(got[~nan]).all()
    err = np.abs(got[~nan].astype(np.float64) - want[~nan]) / (1.0 + np.abs(x[~nan].astype(np.float64)))
    print("%s: worst |d| / (1 + |x|) = %.3g at x = %g" % (kind, err.max(), x[~nan][err.argmax()]))
    assert err.max() <= 4e-7
