"""Edge shapes of the 3x3 convolutions against the CPU oracle: the Winograd
F(2x2, 3x3) kernel (mx_wino3_*, from 8 input channels in multiples of 8 and
32 output channels, widths a multiple of 8), the channel-last kernel (mx_c3_*,
from 128 input channels) and the implicit-GEMM kernel (the rest): image sides
that are not a multiple of the tile, output-channel counts that leave a
partial block, channel counts that leave a partial chunk, both Winograd tile
widths, a fused leaky ReLU, and a misaligned output.
GEMM bar: max|d| <= 1e-4 * max|cpu| (matrix-core reduction order).
"""


def expect_kernel(ci, co, h, w):
    """The executor's choice of 3x3 kernel for an aligned input."""
    if co <= 4 and ci >= 64:
        return "mx_conv3x3_co4"
    if ci >= 8 and ci % 8 == 0 and co >= 32 and w % 8 == 0:
        return "mx_wino3_t16" if w % 32 == 0 else "mx_wino3_t8" if w % 16 == 0 else "mx_wino3_t4"
    if ci % 16 == 0 and ci >= 128:
        return "mx_c3_"
    return "mx_conv3x3v_" if w % 16 == 0 else "mx_conv3x3_"

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
    (24, 16, 8, 16),     # 24 input channels: the implicit-GEMM kernel (vector halo)
    (32, 32, 19, 48),    # vector halo: ragged rows, three column tiles, every border
    (20, 40, 13, 32),    # vector halo: a partial channel chunk and a partial block
    (64, 3, 10, 64),     # three output channels: the vector-ALU kernel
    (70, 3, 13, 21),     # the same with ragged tiles and a channel count off the wave split
    (96, 4, 9, 150),     # four outputs, 4 x 64 tiles ragged in both directions
    (30, 3, 13, 21),     # three outputs from fewer inputs: 16-channel MFMA blocks
    (16, 64, 11, 40),    # Winograd: two chunks, two output blocks, ragged rows
    (24, 40, 9, 16),     # Winograd: three chunks, a partial output block
    (32, 32, 128, 1024), # Winograd with 8 x 16-pixel blocks
    (128, 128, 20, 32),  # Winograd over 16 chunks
    (64, 32, 13, 64),    # Winograd with 4 x 32-pixel blocks, ragged rows
    (32, 64, 18, 48),    # Winograd with 8 x 16-pixel blocks, ragged rows
    (8, 40, 20, 96),     # Winograd, one chunk, a partial second channel block
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
    assert steps[0][2].startswith(expect_kernel(ci, co, h, w))
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
    # the LeakyReLU-only specialisation of the Winograd kernel's epilogue
    assert len(steps) == 1 and steps[0][2].startswith("mx_wino3_") and steps[0][2].endswith("_f_e16")
    check(got, oracle_plan(cp, {0: x}, 3), "conv3x3 + lrelu, output misaligned %d" % misalign)


def unfused(cp, inputs, out):
    from maxim_amd import hip as H
    gpu = H.Gpu(cp)
    gpu.set_fusion(False)
    for b, v in inputs.items():
        gpu.write_buf(b, v)
    gpu.run_ops(0, len(cp.ops))
    got = gpu.read_buf(out).reshape(cp.bufs[out])
    gpu.close()
    return got


@pytest.mark.parametrize("co,h,w", [(32, 12, 32), (64, 9, 21), (128, 8, 20)])
def test_attention_gate_fused(gpu_ok, co, h, w):
    """The supervised attention module's gate, Conv3x3 (3 -> co) -> Sigmoid
    -> Mul -> Add, as one step whose conv epilogue applies all three (128-bit
    operand reads where the rows allow, element by element at a ragged
    edge): the unfused ops' bits, and the CPU path within the GEMM bar."""
    from maxim_amd import plan as P
    rng = np.random.default_rng(co + w)
    img = rng.standard_normal((3, h, w)).astype(np.float32)
    f1 = rng.standard_normal((co, h, w)).astype(np.float32)
    res = rng.standard_normal((co, h, w)).astype(np.float32)
    wt = he(rng, (co, 3, 3, 3), 27)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    n = co * h * w
    bufs = [(3, h, w), (co, h, w), (co, h, w), (co, h, w), (co, h, w), (co, h, w), (co, h, w)]
    ops = [P.make_op(P.CONV3X3, dst=1, src=0, w=0, bias=1, c_in=3, c_out=co, h=h, wd=w),
           P.make_op(P.SIGMOID, dst=2, src=1, n=n),
           P.make_op(P.MUL, dst=4, src=2, src2=3, n=n),
           P.make_op(P.ADD, dst=6, src=4, src2=5, n=n)]
    cp = P.CustomPlan(bufs, ops, [wt, b], input=0, output=6)
    inputs = {0: img, 3: f1, 5: res}
    got, steps = run_plan(cp, inputs, 6)
    print("steps", steps)
    assert len(steps) == 1 and steps[0][2].endswith("_f"), steps
    assert np.array_equal(got.view(np.uint32), unfused(cp, inputs, 6).view(np.uint32))
    check(got, oracle_plan(cp, inputs, 6), "conv3x3 3->%d + sigmoid * f + r @%dx%d" % (co, h, w))


@pytest.mark.parametrize("ci,h,w", [(64, 10, 64), (32, 13, 21)])
def test_conv3x3_add_fused(gpu_ok, ci, h, w):
    """A stage's output image: Conv3x3 (ci -> 3) -> Add (the input image) as
    one step with the add in the conv's epilogue; the unfused bits, and the
    CPU path within the GEMM bar."""
    from maxim_amd import plan as P
    rng = np.random.default_rng(ci + w)
    x = rng.standard_normal((ci, h, w)).astype(np.float32)
    img = rng.standard_normal((3, h, w)).astype(np.float32)
    wt = he(rng, (3, ci, 3, 3), 9 * ci)
    b = (rng.standard_normal(3) * 0.1).astype(np.float32)
    bufs = [(ci, h, w), (3, h, w), (3, h, w), (3, h, w)]
    ops = [P.make_op(P.CONV3X3, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=3, h=h, wd=w),
           P.make_op(P.ADD, dst=3, src=1, src2=2, n=3 * h * w)]
    cp = P.CustomPlan(bufs, ops, [wt, b], input=0, output=3)
    inputs = {0: x, 2: img}
    got, steps = run_plan(cp, inputs, 3)
    print("steps", steps)
    assert len(steps) == 1 and steps[0][2].endswith("_f"), steps
    assert np.array_equal(got.view(np.uint32), unfused(cp, inputs, 3).view(np.uint32))
    check(got, oracle_plan(cp, inputs, 3), "conv3x3 %d->3 + image @%dx%d" % (ci, h, w))


@pytest.mark.parametrize("ci,co,h,w,split", [
    (64, 64, 224, 320, True),    # the C4 112x160 downsampling: 280 blocks, four slices of four chunks
    (128, 128, 112, 160, True),  # the C4 56x80 one: four slices of eight chunks
    (128, 96, 40, 36, True),     # a partial channel block, output rows not a multiple of 4 wide
    (32, 32, 448, 640, False),   # the C4 224x320 one fills the chip unsplit
    (64, 32, 30, 38, False),     # 15x19 outputs: a plane not a multiple of 4
])
def test_conv4x4_split_reduction(gpu_ok, ci, co, h, w, split):
    """4x4 stride-2 convs whose blocks do not fill the chip split the input
    channels over z-slices (partial outputs in scratch) and sum the slices in
    z order with the bias (mx_conv_split_sum); within the GEMM bar of the CPU
    path either way."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    from oracle import oracle as O
    rng = np.random.default_rng(ci + co + h)
    x = rng.standard_normal((ci, h, w)).astype(np.float32)
    wt = he(rng, (co, ci, 4, 4), 16 * ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    pt, _ = P.same_pad(h, 2, 4)
    pl, _ = P.same_pad(w, 2, 4)
    oh, ow = (h + 1) // 2, (w + 1) // 2
    op = P.make_op(P.CONV4X4S2, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=co, h=h, wd=w, oh=oh, ow=ow, p=[pt, pl])
    cp = P.CustomPlan([(ci, h, w), (co, oh, ow)], [op], [wt, b], input=0, output=1)
    gpu = H.Gpu(cp)
    gpu.write_buf(0, x)
    gpu.run_ops(0, 1)
    got = gpu.read_buf(1).reshape(co, oh, ow)
    ks = [k for _, k in gpu.launches()]
    gpu.close()
    print(ks)
    if split:
        assert len(ks) == 2 and ks[0].startswith("mx_conv4x4_") and ks[0].endswith("_s") and ks[1] == "mx_conv_split_sum", ks
    else:
        assert len(ks) == 1 and ks[0].startswith("mx_conv4x4_") and not ks[0].endswith("_s"), ks
    check(got, O.conv4x4s2(x, wt, b, pt, pl), "conv4x4s2 %d->%d @%dx%d" % (ci, co, h, w))
