"""Edge shapes of the channel-last 3x3 convolution (mx_c3_*, used from 128
input channels) against the CPU oracle: image sides that are not a multiple
of the tile (16 columns, 2, 4 or 8 rows), output-channel counts that leave a
partial block, 128 and 256 input channels, a fused leaky ReLU, and the
fallbacks to the implicit-GEMM kernel (fewer input channels; a misaligned
output).
GEMM bar: max|d| <= 1e-4 * max|cpu| (matrix-core reduction order).
"""

import numpy as np
import pytest

from test_gpu_pointwise import check, he, oracle_plan, run_plan

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ci,co,h,w", [
    (128, 128, 20, 28),  # eight chunks, 64-channel blocks of 2 rows, ragged columns
    (128, 192, 9, 20),   # three 64-channel blocks of 2 rows, an odd row count
    (128, 40, 9, 20),    # 32-channel blocks of 8 rows, the second block partial
    (256, 64, 7, 12),    # sixteen chunks, a 12-wide image
    (128, 64, 33, 4),    # a 4-wide image
    (32, 40, 17, 36),    # below 128 input channels: the implicit-GEMM kernel
    (24, 16, 8, 16),     # 24 input channels: the implicit-GEMM kernel
])
def test_conv3x3_edges(gpu_ok, ci, co, h, w):
    from maxim_amd import plan as P
    from oracle import oracle as O
    rng = np.random.default_rng(ci * 7 + co + h)
    x = rng.standard_normal((ci, h, w)).astype(np.float32)
    wt = he(rng, (co, ci, 3, 3), 9 * ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    op = P.make_op(P.CONV3X3, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=co, h=h, wd=w)
    cp = P.CustomPlan([(ci, h, w), (co, h, w)], [op], [wt, b], input=0, output=1)
    got, steps = run_plan(cp, {0: x}, 1)
    print("kernel", steps[0][2])
    assert steps[0][2].startswith("mx_c3_" if ci % 16 == 0 and ci >= 128 else "mx_conv3x3_")
    check(got, O.conv3x3(x, wt, b), "conv3x3 %d->%d @%dx%d" % (ci, co, h, w))


@pytest.mark.parametrize("misalign", [0, 1])
def test_conv3x3_lrelu_fused(gpu_ok, misalign):
    """Conv3x3 -> Lrelu as one step; with the output one float off a 16-byte
    boundary the step falls back to the older kernel's fused form."""
    from maxim_amd import plan as P
    ci, co, h, w = 128, 32, 12, 40
    rng = np.random.default_rng(5 + misalign)
    x = rng.standard_normal((ci, h, w)).astype(np.float32)
    wt = he(rng, (co, ci, 3, 3), 9 * ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    n = co * h * w
    bufs = [(ci, h, w), (co, h, w), (1, 1, 1 if misalign else 4), (co, h, w)]
    ops = [P.make_op(P.CONV3X3, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=co, h=h, wd=w),
           P.make_op(P.LRELU, dst=3, src=1, n=n, slope=0.2)]
    cp = P.CustomPlan(bufs, ops, [wt, b], input=0, output=3, align=1)
    assert (int(cp.offs[3]) % 4 != 0) == bool(misalign)
    got, steps = run_plan(cp, {0: x}, 3)
    print("steps", steps)
    assert len(steps) == 1 and steps[0][2].endswith("_f")
    assert steps[0][2].startswith("mx_conv3x3_" if misalign else "mx_c3_")
    check(got, oracle_plan(cp, {0: x}, 3), "conv3x3 + lrelu, output misaligned %d" % misalign)
