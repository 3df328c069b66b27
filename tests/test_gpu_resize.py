"""Bilinear resize (antialiased on downscale) against the CPU oracle, bit for bit.

The resize op (src/exec_cpu.rs:1195-1260) runs a horizontal then a vertical
pass of tap sums. The executor runs both in one kernel when the taps allow
(mx_resize_hv[4]_t<taps>: a block stages the input rows and columns its outputs
read in LDS and rebuilds the horizontal rows there; 64 or 256 output columns
per block) and as two kernels through the intermediate plane otherwise; all
must match the CPU path exactly, including at ragged widths, odd ratios,
partial tiles and the MAXIM pyramid's x4 / x2 / /2 / /4 steps.
"""

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [
    # c, h, w -> oh, ow
    (4, 28, 40, 112, 160),    # x4 up (pyramid level 2 -> 0)
    (4, 56, 80, 112, 160),    # x2 up
    (3, 112, 160, 28, 40),    # /4 down
    (3, 112, 160, 56, 80),    # /2 down
    (2, 17, 23, 50, 71),      # odd ratios up, widths not multiples of 64
    (2, 50, 71, 17, 23),      # odd ratios down
    (5, 64, 64, 64, 64),      # identity
    (1, 1, 1, 3, 130),        # one input pixel
    (2, 9, 130, 9, 65),       # one axis only
    (2, 30, 70, 60, 300),     # 256-column tiles, the second one partial
    (3, 13, 57, 40, 172),     # odd upsampling ratios, 256-column tiles
]


def run_resize(c, h, w, oh, ow, x, two_pass):
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    op = P.make_op(P.RESIZE, dst=2, src=0, src2=1, c=c, h=h, wd=w, oh=oh, ow=ow)
    cp = P.CustomPlan([(c, h, w), (c, h, ow), (c, oh, ow)], [op], [], input=0, output=2)
    old = os.environ.pop("MAXIM_RESIZE_2PASS", None)
    if two_pass:
        os.environ["MAXIM_RESIZE_2PASS"] = "1"
    try:
        gpu = H.Gpu(cp)
    finally:
        os.environ.pop("MAXIM_RESIZE_2PASS", None)
        if old is not None:
            os.environ["MAXIM_RESIZE_2PASS"] = old
    kernels = [k for _, k in gpu.launches()]
    gpu.write_buf(0, x)
    gpu.step_op(0)
    got = gpu.read_buf(2).reshape(c, oh, ow)
    gpu.close()
    return got, kernels


@pytest.mark.parametrize("two_pass", [False, True], ids=["one_pass", "two_pass"])
@pytest.mark.parametrize("c,h,w,oh,ow", CASES)
def test_resize_bit_exact(gpu_ok, c, h, w, oh, ow, two_pass):
    from oracle import oracle as O
    print("resize %dx%dx%d -> %dx%d %s" % (c, h, w, oh, ow, "two-pass" if two_pass else "one-pass"),
          flush=True)
    rng = np.random.default_rng(h * 1000 + w)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    got, kernels = run_resize(c, h, w, oh, ow, x, two_pass)
    want = O.resize(x, oh, ow)
    if two_pass:
        assert kernels == ["mx_resize_h", "mx_resize_v"], kernels
    else:
        # 256-column tiles where the columns are not downsampled and ow % 4 == 0
        kern = "mx_resize_hv4_t" if ow >= w and ow % 4 == 0 else "mx_resize_hv_t"
        assert len(kernels) == 1 and kernels[0].startswith(kern), kernels
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        float(np.abs(got.astype(np.float64) - want).max())


def test_resize_pyramid_shapes(gpu_ok):
    """The C4 pyramid's full-size steps (c reduced), one-pass, bit-exact."""
    from oracle import oracle as O
    rng = np.random.default_rng(7)
    for (c, h, w, oh, ow) in [(2, 112, 160, 448, 640), (2, 448, 640, 112, 160),
                              (2, 224, 320, 448, 640), (2, 448, 640, 224, 320)]:
        print("resize %dx%dx%d -> %dx%d" % (c, h, w, oh, ow), flush=True)
        x = rng.standard_normal((c, h, w)).astype(np.float32)
        got, kernels = run_resize(c, h, w, oh, ow, x, False)
        assert len(kernels) == 1 and kernels[0].startswith("mx_resize_hv4_t" if ow > w else "mx_resize_hv_t"), kernels
        want = O.resize(x, oh, ow)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
