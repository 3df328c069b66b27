"""The two rules that reorder arithmetic (MAXIM_PLAN_ORDER=1 turns both off).

Upsampling Resize -> 1x1 conv (the reference's UpSampleRatio,
src/model.rs builds it as a Resize op followed by a Conv1x1 op) run in the
other order: the conv at the resize's input resolution, then the resize of
the conv's fewer channels.

Both ops are linear; the resize mixes pixels of one channel plane with taps
that sum to one, the conv mixes channels of one pixel, so
W R(x) + b = R(W x + b) up to rounding. The tests pin:
- which pairs the executor commutes (upsampling, fewer outputs than inputs,
  the resize output read by the conv alone) and which it leaves alone;
- the commuted pair against the plan's own order on the device (rounding
  only: 4e-6 of the output's magnitude) and against the CPU path at the GEMM
  bar (1e-4 * max|cpu|);
- MAXIM_PLAN_ORDER=1 restores the plan's order: fused = unfused to the bit.
"""

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [
    # c_in, h, w -> oh, ow, c_out, commuted
    (64, 112, 160, 224, 320, 32, True),   # x2 (the C4 decoder's 224x320 -> 448x640 step, 1/2 size)
    (128, 28, 40, 112, 160, 32, True),    # x4
    (64, 30, 44, 60, 88, 48, True),       # x2, widths not multiples of 64
    (32, 56, 80, 112, 160, 64, False),    # more outputs than inputs: the plan's order is cheaper
    (64, 112, 160, 56, 80, 16, False),    # downsampling
]


def pair_plan(ci, h, w, oh, ow, co, seed):
    from maxim_amd import plan as P
    rng = np.random.default_rng(seed)
    wt = (rng.standard_normal((co, ci)) * np.sqrt(2.0 / ci)).astype(np.float32)
    b = rng.normal(0, 0.1, co).astype(np.float32)
    ops = [P.make_op(P.RESIZE, dst=2, src=0, src2=1, c=ci, h=h, wd=w, oh=oh, ow=ow),
           P.make_op(P.CONV1X1, dst=3, src=2, w=0, bias=1, c_in=ci, c_out=co, h=oh, wd=ow)]
    bufs = [(ci, h, w), (ci, h, ow), (ci, oh, ow), (co, oh, ow)]
    cp = P.CustomPlan(bufs, ops, [wt.ravel(), b], input=0, output=3)
    x = rng.standard_normal((ci, h, w)).astype(np.float32)
    return cp, x


def run(cp, x, fused, no_commute=False):
    from maxim_amd import hip as H
    old = os.environ.pop("MAXIM_PLAN_ORDER", None)
    if no_commute:
        os.environ["MAXIM_PLAN_ORDER"] = "1"
    try:
        gpu = H.Gpu(cp)
    finally:
        os.environ.pop("MAXIM_PLAN_ORDER", None)
        if old is not None:
            os.environ["MAXIM_PLAN_ORDER"] = old
    gpu.set_fusion(fused)
    gpu.write_buf(0, x)
    gpu.run_ops(0, len(cp.ops))
    out = gpu.read_buf(3).reshape(cp.bufs[3])
    kernels = [k for _, k in gpu.launches()]
    gpu.close()
    return out, kernels


@pytest.mark.parametrize("ci,h,w,oh,ow,co,commuted", CASES)
def test_upsample_conv_commuted(gpu_ok, ci, h, w, oh, ow, co, commuted):
    from oracle import oracle as O
    cp, x = pair_plan(ci, h, w, oh, ow, co, seed=ci + h + co)
    fused, kernels = run(cp, x, True)
    plain, plain_k = run(cp, x, False)
    print("%dx%dx%d -> %dx%d, %d -> %d: %s" % (ci, h, w, oh, ow, ci, co, kernels), flush=True)
    if commuted:
        assert kernels[0].startswith("mx_pw_") and kernels[1].startswith("mx_resize_hv"), kernels
    else:
        assert kernels == plain_k and kernels[0].startswith("mx_resize"), kernels
    arena = np.zeros(cp.arena_len, np.float32)
    arena[:x.size] = x.ravel()
    O.run(cp, arena)
    o = int(cp.offs[3])
    ref = arena[o:o + co * oh * ow].reshape(co, oh, ow).astype(np.float64)
    scale = float(np.abs(ref).max())
    d_plain = float(np.abs(fused.astype(np.float64) - plain).max())
    d_cpu = float(np.abs(fused.astype(np.float64) - ref).max())
    print("max|cpu| %.3g: fused vs plan order %.3g, fused vs CPU %.3g, plan order vs CPU %.3g"
          % (scale, d_plain, d_cpu, float(np.abs(plain.astype(np.float64) - ref).max())), flush=True)
    assert np.isfinite(fused).all()
    assert d_plain <= 4e-6 * scale
    assert d_cpu <= 1e-4 * scale
    if not commuted:
        assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    # with the switch, the fused program keeps the plan's order and its bits
    kept, kept_k = run(cp, x, True, no_commute=True)
    assert kept_k[0].startswith("mx_resize")
    assert np.array_equal(kept.view(np.uint32), plain.view(np.uint32))


def test_c4_pairs_commuted(gpu_ok):
    """At C4 every UpSampleRatio whose resize upsamples runs commuted (18 of
    the 36 resizes; the other 18 downsample), and the pass stays within the
    whole-pass bar of the plan's order."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    from conftest import smooth_image, weights
    plan = P.Plan(weights("S-3"), 448, 640)
    img = smooth_image(448, 640, seed=22)
    gpu = H.Gpu(plan)
    steps = gpu.steps()
    com = [(a, b) for a, b, k in steps if plan.ops[a].kind == P.RESIZE and b == a + 2 and k.startswith("mx_pw_")]
    ups = [i for i, o in enumerate(plan.ops) if o.kind == P.RESIZE and o.oh * o.ow > o.h * o.wd]
    print("%d commuted pairs, %d upsampling resizes, %d resizes" %
          (len(com), len(ups), sum(o.kind == P.RESIZE for o in plan.ops)), flush=True)
    assert len(com) == len(ups) == 18
    got = gpu.run(img).copy()
    gpu.set_fusion(False)
    plain = gpu.run(img)
    gpu.close()
    d = float(np.abs(got.astype(np.float64) - plain).max())
    print("fused (commuted) vs op by op: max-abs %.3g" % d)
    assert d <= 2e-5


def test_cut_inside_commuted_pair(gpu_ok):
    """A run of ops that ends between the resize and the conv runs the pair
    in the plan's order (the resize's output is materialised), so the pass in
    two pieces equals the op-by-op pass to the bit."""
    from maxim_amd import hip as H
    cp, x = pair_plan(64, 56, 80, 112, 160, 16, seed=5)
    plain, _ = run(cp, x, False)
    gpu = H.Gpu(cp)
    assert [k for _, k in gpu.launches()][0].startswith("mx_pw_")
    gpu.write_buf(0, x)
    gpu.run_ops(0, 1)
    gpu.run_ops(1, 2)
    got = gpu.read_buf(3).reshape(cp.bufs[3])
    gpu.close()
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32))


@pytest.mark.parametrize("h,w", [(56, 80), (30, 44)])
def test_split_gemm_layernorm_statistics(gpu_ok, h, w):
    """ChanLn over 128 channels -> 1x1 conv with the split reduction: the
    GEMM forms each pixel's statistics from the channels its block's four
    waves hold (the _k4_ln2 kernels, no statistics pass). Against the CPU
    path at the GEMM bar, inputs with a per-pixel offset of 3 and spread 0.5
    (so the one-pass variance matters), plane sizes with and without a
    ragged last tile; MAXIM_PLAN_ORDER=1 restores the statistics pass and
    the unfused bits."""
    from maxim_amd import plan as P
    from oracle import oracle as O
    rng = np.random.default_rng(h + w)
    c, co = 128, 96
    x = (3.0 + 0.5 * rng.standard_normal((c, h, w)) + rng.standard_normal((1, h, w))).astype(np.float32)
    scale = rng.normal(1.0, 0.1, c).astype(np.float32)
    shift = rng.normal(0.0, 0.1, c).astype(np.float32)
    wt = (rng.standard_normal((co, c)) * np.sqrt(2.0 / c)).astype(np.float32)
    b = rng.normal(0, 0.1, co).astype(np.float32)
    ops = [P.make_op(P.CHAN_LN, dst=1, src=0, scale=0, bias=1, c=c, hw=h * w),
           P.make_op(P.CONV1X1, dst=2, src=1, w=2, bias=3, c_in=c, c_out=co, h=h, wd=w)]
    cp = P.CustomPlan([(c, h, w), (c, h, w), (co, h, w)], ops, [scale, shift, wt.ravel(), b], input=0, output=2)

    def go(fused, plan_order=False):
        from maxim_amd import hip as H
        old = os.environ.pop("MAXIM_PLAN_ORDER", None)
        if plan_order:
            os.environ["MAXIM_PLAN_ORDER"] = "1"
        try:
            gpu = H.Gpu(cp)
        finally:
            os.environ.pop("MAXIM_PLAN_ORDER", None)
            if old is not None:
                os.environ["MAXIM_PLAN_ORDER"] = old
        gpu.set_fusion(fused)
        gpu.write_buf(0, x)
        gpu.run_ops(0, 2)
        out = gpu.read_buf(2).reshape(co, h, w)
        ks = [k for _, k in gpu.launches()]
        gpu.close()
        return out, ks

    got, ks = go(True)
    print(ks)
    assert any(k.startswith("mx_pw_ch2_k4_ln2") for k in ks) and not any(k.startswith("mx_chan_ln") for k in ks), ks
    arena = np.zeros(cp.arena_len, np.float32)
    arena[:x.size] = x.ravel()
    O.run(cp, arena)
    o = int(cp.offs[2])
    ref = arena[o:o + co * h * w].reshape(co, h, w).astype(np.float64)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    print("max|cpu| %.3g, max-abs %.3g" % (float(np.abs(ref).max()), err))
    assert np.isfinite(got).all() and err <= 1e-4 * float(np.abs(ref).max())
    kept, ks2 = go(True, plan_order=True)
    plain, _ = go(False)
    assert any(k.startswith("mx_chan_ln_stats") for k in ks2), ks2
    assert np.array_equal(kept.view(np.uint32), plain.view(np.uint32))


def test_commuted_pair_into_a_misaligned_output(gpu_ok):
    """The commuted pair's resize writes the conv's output, and the 256-column
    resize stores 128 bits: with that output one float off a 16-byte
    boundary the pair runs in the plan's order instead (the plan-order resize
    writes its own, aligned output), bit-equal to the op-by-op pass and within
    the GEMM bar of the CPU path."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    from oracle import oracle as O
    ci, h, w, oh, ow, co = 64, 30, 44, 60, 88, 16
    rng = np.random.default_rng(9)
    wt = (rng.standard_normal((co, ci)) * np.sqrt(2.0 / ci)).astype(np.float32)
    b = rng.normal(0, 0.1, co).astype(np.float32)
    ops = [P.make_op(P.RESIZE, dst=2, src=0, src2=1, c=ci, h=h, wd=w, oh=oh, ow=ow),
           P.make_op(P.CONV1X1, dst=4, src=2, w=0, bias=1, c_in=ci, c_out=co, h=oh, wd=ow)]
    bufs = [(ci, h, w), (ci, h, ow), (ci, oh, ow), (1, 1, 1), (co, oh, ow)]
    cp = P.CustomPlan(bufs, ops, [wt.ravel(), b], input=0, output=4, align=1)
    assert int(cp.offs[2]) % 4 == 0 and int(cp.offs[4]) % 4 == 1
    x = rng.standard_normal((ci, h, w)).astype(np.float32)
    out = {}
    for fused in (True, False):
        gpu = H.Gpu(cp)
        assert gpu.buf_offset(4) % 4 == 1  # elements: 4 bytes past a 16-byte boundary
        gpu.set_fusion(fused)
        gpu.write_buf(0, x)
        gpu.run_ops(0, len(cp.ops))
        out[fused] = (gpu.read_buf(4).reshape(co, oh, ow), [k for _, k in gpu.launches()])
        gpu.close()
    got, kernels = out[True]
    print("kernels", kernels, flush=True)
    # the plan's order: the resize first (the conv then takes a kernel that
    # stores to any 4-byte boundary)
    assert len(kernels) == 2 and kernels[0].startswith("mx_resize_hv4_"), kernels
    assert np.array_equal(got.view(np.uint32), out[False][0].view(np.uint32))
    arena = np.zeros(cp.arena_len, np.float32)
    arena[:x.size] = x.ravel()
    O.run(cp, arena)
    o = int(cp.offs[4])
    ref = arena[o:o + co * oh * ow].reshape(co, oh, ow).astype(np.float64)
    assert float(np.abs(got - ref).max()) <= 1e-4 * float(np.abs(ref).max())
