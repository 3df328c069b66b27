"""The isolated benchmark configurations, each against the CPU oracle.

C2: one multi-axis gated-MLP layer (ResidualSplitHeadMultiAxisGmlpLayer,
    src/model.rs:576-603) at c = 32, 256x256, block 16 + grid 16, x ~ N(0, 1):
    the 25 ops from LayerNorm_in to the residual add, taken from the MAXIM-2S
    plan and run on both paths from the same input.
C3: the conv stack at encoder shapes, fp32, pad 1, He-normal weights,
    x ~ N(0, 1): 3x3 32->32 @512^2, 64->64 @256^2, 128->128 @128^2,
    4x4 stride-2 32->64 @512^2, transposed 2x2 stride-2 128->64 @128^2, each a
    one-op plan handed to the executor through the C ABI.
GEMM bar: max|d| <= 1e-4 * max|cpu| (matrix-core reduction order).
"""

import numpy as np
import pytest

from conftest import buf, weights

pytestmark = pytest.mark.gpu


def he(rng, shape, fan_in):
    return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def run_one(op, bufs, wts, x):
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    cp = P.CustomPlan(bufs, [op], wts, input=op.src, output=op.dst)
    gpu = H.Gpu(cp)
    gpu.write_buf(op.src, x)
    gpu.step_op(0)
    return gpu.read_buf(op.dst).reshape(bufs[op.dst])


def check(got, want, label):
    err = float(np.abs(got.astype(np.float64) - want).max())
    scale = float(np.abs(want).max())
    print("%s: max|cpu| %.3g, max-abs %.3g, relative %.3g" % (label, scale, err, err / scale), flush=True)
    assert err <= 1e-4 * scale, label


@pytest.mark.parametrize("ci,co,side", [(32, 32, 512), (64, 64, 256), (128, 128, 128)])
def test_c3_conv3x3(gpu_ok, ci, co, side):
    from maxim_amd import plan as P
    from oracle import oracle as O
    rng = np.random.default_rng(ci)
    x = rng.standard_normal((ci, side, side)).astype(np.float32)
    w = he(rng, (co, ci, 3, 3), 9 * ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    op = P.make_op(P.CONV3X3, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=co, h=side, wd=side)
    got = run_one(op, [(ci, side, side), (co, side, side)], [w, b], x)
    check(got, O.conv3x3(x, w, b), "conv3x3 %d->%d @%d^2" % (ci, co, side))


def test_c3_conv4x4s2(gpu_ok):
    from maxim_amd import plan as P
    from oracle import oracle as O
    ci, co, side = 32, 64, 512
    rng = np.random.default_rng(44)
    x = rng.standard_normal((ci, side, side)).astype(np.float32)
    w = he(rng, (co, ci, 4, 4), 16 * ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    pt, _ = P.same_pad(side, 2, 4)
    op = P.make_op(P.CONV4X4S2, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=co, h=side, wd=side,
                   oh=side // 2, ow=side // 2, p=[pt, pt])
    got = run_one(op, [(ci, side, side), (co, side // 2, side // 2)], [w, b], x)
    check(got, O.conv4x4s2(x, w, b, pt, pt), "conv4x4s2 %d->%d @%d^2" % (ci, co, side))


def test_c3_convt2x2(gpu_ok):
    from maxim_amd import plan as P
    from oracle import oracle as O
    ci, co, side = 128, 64, 128
    rng = np.random.default_rng(22)
    x = rng.standard_normal((ci, side, side)).astype(np.float32)
    w = he(rng, (ci, co, 2, 2), 4 * ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    op = P.make_op(P.CONVT2X2, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=co, h=side, wd=side)
    got = run_one(op, [(ci, side, side), (co, 2 * side, 2 * side)], [w, b], x)
    check(got, O.convt2x2(x, w, b), "convt2x2 %d->%d @%d^2" % (ci, co, side))


def gmlp_range(plan):
    """Ops of the first split-head gMLP layer: after the encoder's Conv_0,
    through the layer's residual add."""
    from maxim_amd import plan as P
    d = dict(plan.dumps)
    x = d["stage_0_encoder_block_0_mid_conv"]
    y = d["stage_0_encoder_block_0_mid_g0_gmlp"]
    first = next(i for i, op in enumerate(plan.ops) if op.dst == x) + 1
    last = next(i for i, op in enumerate(plan.ops) if op.dst == y) + 1
    return x, y, first, last


def test_c2_gmlp_layer_with_baseline_weights(gpu_ok, tmp_path):
    """C2 as the benchmark defines it: the split-head gMLP layer at c=32,
    256x256, x ~ N(0, 1), with every Dense and LayerNorm parameter of the
    layer ~ N(0, 0.02), written into a checkpoint file and read back through
    the safetensors loader (the variant comes from the file)."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    from oracle import oracle as O
    from conftest import rewrite_safetensors
    path = str(tmp_path / "c2.safetensors")
    weights("S-2").save(path)
    prefix = "stage_0_encoder_block_0/SplitHeadMultiAxisGmlpLayer_0/"
    g = np.random.default_rng(20)
    touched = []

    def n002(name, old):
        if not name.startswith(prefix):
            return None
        touched.append(name)
        return (0.02 * g.standard_normal(old.shape)).astype(np.float32)

    rewrite_safetensors(path, n002)
    assert len(touched) == 26, touched
    w = P.Weights.open(path)
    assert w.config.num_stages == 2 and w.config.features == 32
    plan = P.Plan(w, 256, 256, named=True, deep=True)
    x, y, first, last = gmlp_range(plan)
    assert last - first == 25 and plan.bufs[x] == (32, 256, 256)
    xin = np.random.default_rng(8).standard_normal(plan.buf_len(x)).astype(np.float32)
    arena = np.zeros(plan.arena_len, np.float32)
    arena[int(plan.offs[x]):int(plan.offs[x]) + xin.size] = xin
    O.run_range(plan, arena, first, last)
    gpu = H.Gpu(plan)
    gpu.write_buf(x, xin)
    gpu.run_ops(first, last)
    got = gpu.read_buf(y)
    check(got, buf(plan, arena, y), "C2 gMLP layer c=32 256x256, N(0, 0.02) parameters")


def test_c2_gmlp_layer(gpu_ok):
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    from oracle import oracle as O
    plan = P.Plan(weights("S-2"), 256, 256, named=True, deep=True)
    x, y, first, last = gmlp_range(plan)
    assert last - first == 25 and plan.bufs[x] == (32, 256, 256)
    xin = np.random.default_rng(8).standard_normal(plan.buf_len(x)).astype(np.float32)
    arena = np.zeros(plan.arena_len, np.float32)
    arena[int(plan.offs[x]):int(plan.offs[x]) + xin.size] = xin
    O.run_range(plan, arena, first, last)
    gpu = H.Gpu(plan)
    gpu.write_buf(x, xin)
    gpu.run_ops(first, last)
    got = gpu.read_buf(y)
    check(got, buf(plan, arena, y), "C2 gMLP layer c=32 256x256")


def test_chan_ln_one_pass_variance_on_the_gpu(gpu_ok):
    """The device LayerNorm keeps the reference's one-pass fp32 variance
    (src/exec_cpu.rs:403-406): on pixels where a two-pass variance would
    differ by orders of magnitude it gives the one-pass bits exactly."""
    from maxim_amd import plan as P
    from test_oracle import ln_one_pass_fp32, ln_variance_case
    x, s, b = ln_variance_case()
    c, h, w = x.shape
    op = P.make_op(P.CHAN_LN, dst=1, src=0, scale=0, bias=1, c=c, hw=h * w)
    got = run_one(op, [(c, h, w), (c, h, w)], [s, b], x)
    want = ln_one_pass_fp32(x, s, b)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
