"""Edge shapes of the streaming matrix-core kernels (mx_pw_*) against the CPU
oracle, and of the executor's fallback to the tiled GEMM.

The streaming kernels own 64-element tiles of the streamed axis and 16, 32
or 64 weight outputs per wave, and split reductions of 128 and more over a
block's four waves. These cases put every edge inside one op: streamed
lengths that are not a multiple of 64, weight-output counts that leave a
partial block, reductions with and without the split, GateMm in both modes,
a plane that is not a multiple of four (the tiled GEMM takes the op), and
fused epilogues whose extra operand is not 16-byte aligned (the executor
swaps in the tiled kernel's fused form for that step).
GEMM bar: max|d| <= 1e-4 * max|cpu| (matrix-core reduction order).
"""

import re

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def fam(kernel):
    """A kernel's family: the name without the ..._e<mask> suffix of a
    specialisation for one epilogue operand set (same arithmetic)."""
    return re.sub(r"_e\d+$", "", kernel)


def he(rng, shape, fan_in):
    return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)


def check(got, want, label):
    err = float(np.abs(got.astype(np.float64) - want).max())
    scale = float(np.abs(want).max())
    print("%s: max|cpu| %.3g, max-abs %.3g, relative %.3g" % (label, scale, err, err / scale), flush=True)
    assert np.isfinite(got).all(), label
    assert err <= 1e-4 * scale, label


def run_plan(cp, inputs, out):
    """Write every input buffer, run all ops through the fused program,
    return the output buffer and the kernel of each step."""
    from maxim_amd import hip as H
    gpu = H.Gpu(cp)
    for b, v in inputs.items():
        gpu.write_buf(b, v)
    gpu.run_ops(0, len(cp.ops))
    got = gpu.read_buf(out).reshape(cp.bufs[out])
    return got, gpu.steps()


def agree(got, want, order, tol, what):
    """Fused against unfused: the same bits under MAXIM_PLAN_ORDER=1 ("plan");
    in the default order ("free") the LayerNorm statistics of a band held by
    several waves are summed per wave and then across the waves, so the
    outputs agree to rounding (tol, absolute)."""
    if order == "plan":
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "fused and unfused %s differ" % what
    else:
        err = float(np.abs(got.astype(np.float64) - want).max())
        print("%s: fused vs unfused max-abs %.3g (default order)" % (what, err))
        assert err <= tol, (what, err)


def set_order(monkeypatch, order):
    if order == "plan":
        monkeypatch.setenv("MAXIM_PLAN_ORDER", "1")
    else:
        monkeypatch.delenv("MAXIM_PLAN_ORDER", raising=False)


def oracle_plan(cp, inputs, out):
    from oracle import oracle as O
    arena = np.zeros(cp.arena_len, np.float32)
    for b, v in inputs.items():
        o = int(cp.offs[b])
        arena[o:o + v.size] = v.ravel()
    O.run(cp, arena)
    o = int(cp.offs[out])
    return arena[o:o + cp.buf_len(out)].reshape(cp.bufs[out])


@pytest.mark.parametrize("ci,co,h,w", [
    (16, 40, 12, 20),    # K 16, two weight blocks (the second partial), 240 pixels (ragged)
    (48, 24, 8, 30),     # K 48, one partial 32-wide block
    (192, 64, 10, 26),   # K 192: split reduction, 260 pixels
    (256, 136, 6, 14),   # K 256: 64-wide blocks, the last one 8 wide
    (32, 8, 16, 16),     # 16-wide blocks, half used
    (24, 32, 7, 9),      # 63 pixels: not a multiple of four, tiled GEMM
    (64, 32, 64, 64),    # the level-0 shape class
])
def test_conv1x1_edges(gpu_ok, ci, co, h, w):
    from maxim_amd import plan as P
    from oracle import oracle as O
    rng = np.random.default_rng(ci * 1000 + co)
    x = rng.standard_normal((ci, h, w)).astype(np.float32)
    wt = he(rng, (co, ci), ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    op = P.make_op(P.CONV1X1, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=co, h=h, wd=w)
    cp = P.CustomPlan([(ci, h, w), (co, h, w)], [op], [wt, b], input=0, output=1)
    got, steps = run_plan(cp, {0: x}, 1)
    print("kernel", steps[0][2])
    assert steps[0][2].startswith("mx_pw_" if (h * w) % 4 == 0 else "mx_gemm_")
    check(got, O.conv1x1(x, wt, b), "conv1x1 %d->%d @%dx%d" % (ci, co, h, w))


@pytest.mark.parametrize("c,outer,inner,mode", [
    (3, 64, 20, 0),      # K 64, few tiles: split reduction; 20 columns (ragged)
    (2, 48, 36, 0),      # K 48, 48 outputs (partial block)
    (1, 256, 40, 0),     # K 256, 64-wide blocks
    (3, 20, 64, 1),      # row layout, 60 rows (ragged), K 64
    (2, 36, 48, 1),      # row layout, K 48, 48 columns
    (1, 40, 256, 1),     # row layout, K 256
    (2, 64, 70, 0),      # 70 columns: not a multiple of four, tiled GEMM
])
def test_gate_mm_edges(gpu_ok, c, outer, inner, mode):
    from maxim_amd import plan as P
    from oracle import oracle as O
    rng = np.random.default_rng(c * 100 + outer + inner + mode)
    k = outer if mode == 0 else inner
    x = rng.standard_normal((c, outer, inner)).astype(np.float32)
    wt = he(rng, (k, k), k)
    b = (rng.standard_normal(k) * 0.1).astype(np.float32)
    op = P.make_op(P.GATE_MM, dst=1, src=0, w=0, bias=1, c=c, mode=mode, p=[outer, inner])
    cp = P.CustomPlan([(c, outer, inner), (c, outer, inner)], [op], [wt, b], input=0, output=1)
    got, steps = run_plan(cp, {0: x}, 1)
    print("kernel", steps[0][2])
    assert steps[0][2].startswith("mx_pw_" if inner % 4 == 0 else "mx_gemm_")
    check(got, O.gate_mm(x, wt, b, mode), "gate_mm c=%d %dx%d mode %d" % (c, outer, inner, mode))


def fused_case(kind, misalign):
    """conv1x1 feeding GELU or a residual add, or GateMm feeding the gate
    multiply; with `misalign` the epilogue's extra operand (R) starts one
    float past a 16-byte boundary. Buffers: X, pad, R, pad, T, Y."""
    from maxim_amd import plan as P
    rng = np.random.default_rng(7 + misalign)
    if kind == "gate":
        c, outer, inner = 8, 32, 40          # mode 0: K = 32 over 40 columns
        xs = ys = (c, outer, inner)
    else:
        ci, co, h, w = 32, 64, 8, 40
        xs, ys = (ci, h, w), (co, h, w)
    bufs = [xs, (1, 1, 1 if misalign else 4), ys, (1, 1, 3 if misalign else 4), ys, ys]
    X, R, T, Y = 0, 2, 4, 5
    n = ys[0] * ys[1] * ys[2]
    inputs = {X: rng.standard_normal(xs).astype(np.float32),
              R: rng.standard_normal(ys).astype(np.float32)}
    if kind == "gate":
        wt = he(rng, (outer, outer), outer)
        b = (rng.standard_normal(outer) * 0.1).astype(np.float32)
        ops = [P.make_op(P.GATE_MM, dst=T, src=X, w=0, bias=1, c=c, mode=0, p=[outer, inner]),
               P.make_op(P.GATE_APPLY, dst=Y, src=R, src2=T, n=n)]
    else:
        wt = he(rng, (co, ci), ci)
        b = (rng.standard_normal(co) * 0.1).astype(np.float32)
        conv = P.make_op(P.CONV1X1, dst=T, src=X, w=0, bias=1, c_in=ci, c_out=co, h=h, wd=w)
        if kind == "gelu":
            ops = [conv, P.make_op(P.GELU, dst=Y, src=T, n=n)]
        else:
            ops = [conv, P.make_op(P.ADD, dst=Y, src=T, src2=R, n=n)]
    cp = P.CustomPlan(bufs, ops, [wt, b], input=X, output=Y, align=1)
    return cp, inputs, Y


@pytest.mark.parametrize("kind", ["gelu", "add", "gate"])
@pytest.mark.parametrize("misalign", [0, 1])
def test_fused_epilogue_alignment(gpu_ok, kind, misalign):
    cp, inputs, Y = fused_case(kind, misalign)
    r_off = int(cp.offs[2])
    assert (r_off % 4 != 0) == bool(misalign) and int(cp.offs[4]) % 4 == 0
    got, steps = run_plan(cp, inputs, Y)
    print("steps", steps)
    assert len(steps) == 1, "the pair did not fuse"
    kern = fam(steps[0][2])
    assert kern.endswith("_f")
    if misalign and kind != "gelu":
        assert kern.startswith("mx_gemm_"), kern   # 128-bit epilogue loads need alignment
    else:
        assert kern.startswith("mx_pw_"), kern
    want = oracle_plan(cp, inputs, Y)
    check(got, want, "fused %s, operand misaligned %d" % (kind, misalign))


@pytest.mark.parametrize("c,co,h,w,act", [
    (32, 64, 8, 30, True),     # 240 pixels (ragged), GELU epilogue too
    (48, 24, 6, 10, False),    # K 48
    (128, 256, 8, 16, True),   # K 128: split reduction
    (32, 32, 5, 7, False),     # 35 pixels: not folded, the LayerNorm runs on its own
])
def test_layernorm_folded_into_the_dense(gpu_ok, c, co, h, w, act):
    """ChanLn -> Conv1x1 [-> Gelu] as one step: a statistics pass, then the
    streaming GEMM normalising its operand on the way in. Compared with the
    CPU path; the whole-model tests check it is bitwise the unfused pass."""
    from maxim_amd import plan as P
    rng = np.random.default_rng(c + co + h)
    hw = h * w
    x = (rng.standard_normal((c, h, w)) * 2.0 + 0.5).astype(np.float32)
    scale = (1.0 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(c)).astype(np.float32)
    wt = he(rng, (co, c), c)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    ops = [P.make_op(P.CHAN_LN, dst=1, src=0, scale=0, bias=1, c=c, hw=hw),
           P.make_op(P.CONV1X1, dst=2, src=1, w=2, bias=3, c_in=c, c_out=co, h=h, wd=w)]
    bufs = [(c, h, w), (c, h, w), (co, h, w)]
    if act:
        ops.append(P.make_op(P.GELU, dst=3, src=2, n=co * hw))
        bufs.append((co, h, w))
    out = len(bufs) - 1
    cp = P.CustomPlan(bufs, ops, [scale, bias, wt, b], input=0, output=out)
    got, steps = run_plan(cp, {0: x}, out)
    print("steps", steps)
    if hw % 4 == 0:
        assert len(steps) == 1 and "_ln" in steps[0][2], steps
    else:
        assert [(a, b) for a, b, _ in steps] == [(0, 1), (1, 2)], steps
    check(got, oracle_plan(cp, {0: x}, out), "ln %d -> conv1x1 %d->%d @%dx%d%s" % (c, c, co, h, w, " + gelu" if act else ""))


def perm_case(kind, fw, misalign=False):
    """A producer whose output a backward BlockPerm (src/model.rs:104-106)
    scatters to the image: conv1x1 + residual add, or GateMm mode 0 / 1 over
    the blocked tensor. Buffers: X, R, T, S, pad, Y (the image)."""
    from maxim_amd import plan as P
    gh, gw, fh = 4, 4, 8  # 16 cells: GateMm mode 0 reduces over 16
    h, w = gh * fh, gw * fw
    G, Pp = gh * gw, fh * fw
    rng = np.random.default_rng(fw + len(kind) + misalign)
    c = 16 if kind != "conv" else 32
    bl = (c, G, Pp)
    bufs = [bl, bl, bl, bl, (1, 1, 1 if misalign else 4), (c, h, w)]
    X, R, T, S, Y = 0, 1, 2, 3, 5
    inputs = {X: rng.standard_normal(bl).astype(np.float32), R: rng.standard_normal(bl).astype(np.float32)}
    perm = P.make_op(P.BLOCK_PERM, dst=Y, src=S, c=c, h=h, wd=w, mode=0, p=[gh, gw, fh, fw])
    if kind == "conv":
        wt = he(rng, (c, c), c)
        b = (rng.standard_normal(c) * 0.1).astype(np.float32)
        ops = [P.make_op(P.CONV1X1, dst=T, src=X, w=0, bias=1, c_in=c, c_out=c, h=G, wd=Pp),
               P.make_op(P.ADD, dst=S, src=T, src2=R, n=c * G * Pp), perm]
    else:
        mode = 0 if kind == "gate0" else 1
        k = G if mode == 0 else Pp
        wt = he(rng, (k, k), k)
        b = (rng.standard_normal(k) * 0.1).astype(np.float32)
        ops = [P.make_op(P.GATE_MM, dst=S, src=X, w=0, bias=1, c=c, mode=mode, p=[G, Pp]), perm]
    cp = P.CustomPlan(bufs, ops, [wt, b], input=X, output=Y, align=1)
    return cp, inputs, Y


@pytest.mark.parametrize("kind,fw,misalign", [
    ("conv", 8, False), ("gate0", 8, False), ("gate1", 8, False),   # folded into the stores
    ("conv", 12, False), ("gate1", 16, False),
    ("conv", 6, False), ("gate0", 10, False),                       # cells not a multiple of 4 wide
    ("conv", 8, True), ("gate0", 8, True),                          # image one float off 16 bytes
])
def test_block_permutation_folded_into_the_stores(gpu_ok, kind, fw, misalign):
    cp, inputs, Y = perm_case(kind, fw, misalign)
    assert (int(cp.offs[Y]) % 4 != 0) == misalign
    got, steps = run_plan(cp, inputs, Y)
    print("steps", steps)
    n = len(cp.ops)
    if fw % 4 == 0:
        assert len(steps) == 1 and (steps[0][0], steps[0][1]) == (0, n), steps
        assert steps[0][2].startswith("mx_pw_") or misalign
    else:
        assert steps[-1][:2] == (n - 1, n) and steps[-1][2].startswith("mx_block_perm"), steps
    check(got, oracle_plan(cp, inputs, Y), "%s -> block_perm, fw %d, misaligned %d" % (kind, fw, misalign))


def elide_case(kind, gh, gw, fh, fw, c=32):
    """A forward BlockPerm S -> P whose readers take S in image order through
    the block map, so the permutation launches nothing:
      "ln"    the gMLP branch: P -> LayerNorm -> conv1x1 -> gelu -> conv1x1
              + P (residual) -> backward BlockPerm into S, then S copied out;
      "gate0" / "gate1"  the cross-gating: P -> GateMm (mode 0 / 1) ->
              backward BlockPerm to the image."""
    from maxim_amd import plan as P
    h, w = gh * fh, gw * fw
    G, Pp = gh * gw, fh * fw
    rng = np.random.default_rng(gh * 100 + fw + len(kind))
    img, bl = (c, h, w), (c, G, Pp)
    x = rng.standard_normal(img).astype(np.float32)
    fwd = dict(c=c, h=h, wd=w, mode=P.PERM_FORWARD, p=[gh, gw, fh, fw])
    bwd = dict(c=c, h=h, wd=w, mode=0, p=[gh, gw, fh, fw])
    if kind == "ln":
        c2, n = 2 * c, c * G * Pp
        bufs = [img, bl, bl, (c2, G, Pp), (c2, G, Pp), bl, bl, img]
        S, Pb, L, T, U, V, Z, O = range(8)
        wts = [(1.0 + 0.1 * rng.standard_normal(c)).astype(np.float32), (0.1 * rng.standard_normal(c)).astype(np.float32),
               he(rng, (c2, c), c), (0.1 * rng.standard_normal(c2)).astype(np.float32),
               he(rng, (c, c2), c2), (0.1 * rng.standard_normal(c)).astype(np.float32)]
        ops = [P.make_op(P.BLOCK_PERM, dst=Pb, src=S, **fwd),
               P.make_op(P.CHAN_LN, dst=L, src=Pb, scale=0, bias=1, c=c, hw=G * Pp),
               P.make_op(P.CONV1X1, dst=T, src=L, w=2, bias=3, c_in=c, c_out=c2, h=G, wd=Pp),
               P.make_op(P.GELU, dst=U, src=T, n=2 * n),
               P.make_op(P.CONV1X1, dst=V, src=U, w=4, bias=5, c_in=c2, c_out=c, h=G, wd=Pp),
               P.make_op(P.ADD, dst=Z, src=V, src2=Pb, n=n),
               P.make_op(P.BLOCK_PERM, dst=S, src=Z, **bwd),
               P.make_op(P.COPY, dst=O, src=S, n=n)]
    else:
        mode = 0 if kind == "gate0" else 1
        k = G if mode == 0 else Pp
        bufs = [img, bl, bl, img]
        S, Pb, T, O = range(4)
        wts = [he(rng, (k, k), k), (rng.standard_normal(k) * 0.1).astype(np.float32)]
        ops = [P.make_op(P.BLOCK_PERM, dst=Pb, src=S, **fwd),
               P.make_op(P.GATE_MM, dst=T, src=Pb, w=0, bias=1, c=c, mode=mode, p=[G, Pp]),
               P.make_op(P.BLOCK_PERM, dst=O, src=T, **bwd)]
    cp = P.CustomPlan(bufs, ops, wts, input=S, output=O)
    return cp, {S: x}, O


@pytest.mark.parametrize("kind,gh,gw,fh,fw", [
    ("ln", 4, 4, 8, 8),        # 16 cells of 8x8 (the low-resolution block gMLP)
    ("ln", 2, 2, 12, 20),      # grid gMLP shape class: cells 12x20
    ("ln", 3, 5, 4, 12),       # 15 cells, 48-pixel cells: ragged tiles
    ("gate0", 16, 16, 2, 4),   # mode 0 over 256 cells (16 k's = one cell row)
    ("gate0", 8, 8, 3, 8),     # 8-wide grid: 16 k's = two cell rows
    ("gate1", 5, 7, 16, 16),   # mode 1 over 16x16 cells
    ("gate1", 6, 4, 8, 8),     # 8x8 cells: 16 k's = two pixel rows
])
def test_forward_permutation_elided(gpu_ok, kind, gh, gw, fh, fw):
    """The permutation's step launches nothing; the result matches the CPU
    path and is bitwise the unfused pass (which runs the permutation)."""
    from maxim_amd import hip as H
    cp, inputs, out = elide_case(kind, gh, gw, fh, fw)
    got, steps = run_plan(cp, inputs, out)
    print("steps", steps)
    gpu = H.Gpu(cp)
    kern = {st: k for st, k in gpu.launches()}
    first = [s for s, (a, b, _) in enumerate(steps) if a == 0][0]
    assert first not in kern, "the forward permutation still launches: %s" % steps
    assert any(fam(k).endswith(("_xm", "_xm_f")) or "_ln" in k for k in kern.values()), kern
    for b, v in inputs.items():
        gpu.write_buf(b, v)
    gpu.set_fusion(False)
    gpu.run_ops(0, len(cp.ops))
    plain = gpu.read_buf(out).reshape(got.shape)
    gpu.close()
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32)), "fused and unfused passes differ"
    check(got, oracle_plan(cp, inputs, out), "%s perm elided %dx%d cells of %dx%d" % (kind, gh, gw, fh, fw))


@pytest.mark.parametrize("ci,co,h,w,add", [
    (32, 32, 16, 20, True),     # the cross-gating shape class: Mul -> conv1x1 + residual
    (128, 128, 7, 12, False),   # K 128: split reduction, 84 pixels (ragged tile)
    (64, 48, 5, 8, True),
])
def test_mul_folded_into_the_dense(gpu_ok, ci, co, h, w, add):
    """Mul -> Conv1x1 [-> Add] as one streaming launch that multiplies the two
    factors on the way into the GEMM: the CPU path's result to the GEMM bar,
    and bitwise the unfused pass."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    rng = np.random.default_rng(ci + co + h + w)
    n = ci * h * w
    A, B, M_, T, R, Y = range(6)
    bufs = [(ci, h, w), (ci, h, w), (ci, h, w), (co, h, w), (co, h, w), (co, h, w)]
    ops = [P.make_op(P.MUL, dst=M_, src=A, src2=B, n=n),
           P.make_op(P.CONV1X1, dst=T, src=M_, w=0, bias=1, c_in=ci, c_out=co, h=h, wd=w)]
    if add:
        ops.append(P.make_op(P.ADD, dst=Y, src=T, src2=R, n=co * h * w))
    out = Y if add else T
    wt = he(rng, (co, ci), ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    cp = P.CustomPlan(bufs, ops, [wt, b], input=A, output=out)
    inputs = {A: rng.standard_normal(bufs[A]).astype(np.float32), B: rng.standard_normal(bufs[B]).astype(np.float32),
              R: rng.standard_normal(bufs[R]).astype(np.float32)}
    got, steps = run_plan(cp, inputs, out)
    print("steps", steps)
    assert len(steps) == 1 and "_mul" in steps[0][2], steps
    gpu = H.Gpu(cp)
    for k, v in inputs.items():
        gpu.write_buf(k, v)
    gpu.set_fusion(False)
    gpu.run_ops(0, len(cp.ops))
    plain = gpu.read_buf(out).reshape(got.shape)
    gpu.close()
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32)), "fused and unfused passes differ"
    check(got, oracle_plan(cp, inputs, out), "mul -> conv1x1 %d->%d @%dx%d%s" % (ci, co, h, w, " + add" if add else ""))


@pytest.mark.parametrize("ci,co,h,w", [
    (128, 64, 12, 20),   # streaming _t form, split reduction
    (64, 32, 7, 8),      # 56 pixels: one partial tile
    (32, 48, 4, 12),     # 192 rows (ky, oc, kx): a partial weight block
    (32, 16, 5, 6),      # width not a multiple of 4: the tiled GEMM's scatter
    (24, 8, 4, 8),       # K 24: the tiled GEMM
])
def test_transposed_conv_edges(gpu_ok, ci, co, h, w):
    """ConvT 2x2 stride 2 (src/exec_cpu.rs:846-914) on the streaming kernels
    (row order (ky, oc, kx), each lane pair storing eight contiguous outputs)
    and on the tiled fallback, against the CPU path."""
    from maxim_amd import plan as P
    from oracle import oracle as O
    rng = np.random.default_rng(ci * 7 + co + h * w)
    x = rng.standard_normal((ci, h, w)).astype(np.float32)
    wt = he(rng, (ci, co, 2, 2), ci)
    b = (rng.standard_normal(co) * 0.1).astype(np.float32)
    op = P.make_op(P.CONVT2X2, dst=1, src=0, w=0, bias=1, c_in=ci, c_out=co, h=h, wd=w)
    cp = P.CustomPlan([(ci, h, w), (co, 2 * h, 2 * w)], [op], [wt, b], input=0, output=1)
    got, steps = run_plan(cp, {0: x}, 1)
    print("steps", steps)
    streaming = w % 4 == 0 and ci % 16 == 0
    assert steps[0][2].startswith("mx_pw_ch" if streaming else "mx_gemm_") and steps[0][2].endswith("_t"), steps
    check(got, O.convt2x2(x, wt, b), "convt %d->%d @%dx%d" % (ci, co, h, w))


@pytest.mark.parametrize("c,h,w,ln_in", [
    (32, 16, 40, False),   # level-0 gate: c -> 2c + GELU, LayerNorm of the v half
    (32, 12, 52, True),    # with the input LayerNorm folded too (the real level-0 step)
    (64, 8, 36, True),     # 64 channels, few tiles (split reduction): one 64-wide wave
    (64, 128, 256, True),  # 64 channels, 2048 tiles: two 32-wide waves of a block per pixel tile
    (128, 128, 128, False),  # 128 channels, K 128, 2048 tiles: four waves of a block, the reduction kept whole
    (128, 32, 64, False),  # 128 channels, 256 tiles: split reduction kept, the LayerNorm on its own
    (64, 130, 260, False),  # 33800 pixels: a partial last tile for a two-wave group
    (32, 5, 28, False),    # 140 pixels: the last 64-pixel tile partial
])
@pytest.mark.parametrize("order", ["plan", "free"])
def test_layernorm_of_the_gate_half_in_the_epilogue(gpu_ok, monkeypatch, order, c, h, w, ln_in):
    """[ChanLn ->] Conv1x1 c->2c -> Gelu -> ChanLn of channels c..2c (a view):
    one streaming launch whose v-half waves normalise their tile and store only
    the LayerNorm (nothing else reads the raw half). Bitwise the unfused pass
    (the LayerNorm's own order and expression) under MAXIM_PLAN_ORDER=1, to
    rounding in the default order; the CPU path to the GEMM bar."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    set_order(monkeypatch, order)
    rng = np.random.default_rng(c * 100 + h + w)
    hw = h * w
    X, XN, T, G, V, LN = range(6)
    bufs = [(c, h, w), (c, h, w), (2 * c, h, w), (2 * c, h, w), (c, h, w), (c, h, w)]
    views = {V: (G, c * hw)}
    wt = he(rng, (2 * c, c), c)
    b = (rng.standard_normal(2 * c) * 0.1).astype(np.float32)
    g1 = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(c)).astype(np.float32)
    g2 = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(c)).astype(np.float32)
    ops = []
    if ln_in:
        ops.append(P.make_op(P.CHAN_LN, dst=XN, src=X, scale=3, bias=4, c=c, hw=hw))
    ops += [P.make_op(P.CONV1X1, dst=T, src=XN if ln_in else X, w=0, bias=1, c_in=c, c_out=2 * c, h=h, wd=w),
            P.make_op(P.GELU, dst=G, src=T, n=2 * c * hw),
            P.make_op(P.CHAN_LN, dst=LN, src=V, scale=5, bias=6, c=c, hw=hw)]
    cp = P.CustomPlan(bufs, ops, [wt, b, np.zeros(1, np.float32), g1, b1, g2, b2], input=X, output=LN, views=views)
    x = rng.standard_normal(bufs[X]).astype(np.float32)
    gpu = H.Gpu(cp)
    gpu.write_buf(X, x)
    gpu.run_ops(0, len(ops))
    steps = gpu.steps()
    got_ln = gpu.read_buf(LN).reshape(bufs[LN])
    got_u = gpu.read_buf(G).reshape(bufs[G])[:c]
    gpu.set_fusion(False)
    gpu.run_ops(0, len(ops))
    plain_ln = gpu.read_buf(LN).reshape(bufs[LN])
    plain_u = gpu.read_buf(G).reshape(bufs[G])[:c]
    gpu.close()
    print("steps", steps)
    if c == 128 and (2 * c // 32) * ((hw + 63) // 64) < 8 * 256:
        kernels = [k for _, k in H.Gpu(cp).launches()]
        assert len(steps) == 1 and kernels[-1].startswith("mx_chan_ln"), kernels
    else:
        assert len(steps) == 1 and fam(steps[0][2]).endswith("_f_lo"), steps
    agree(got_ln, plain_ln, order, 1e-5, "LayerNorm")
    assert np.array_equal(got_u.view(np.uint32), plain_u.view(np.uint32)), "fused and unfused u half differ"
    want_ln = oracle_plan(cp, {X: x}, LN)
    want_g = oracle_plan(cp, {X: x}, G)
    check(got_u, want_g[:c], "u half c=%d @%dx%d" % (c, h, w))
    # the LayerNorm scales the GEMM's rounding by 1/std of each pixel: an
    # absolute bar on its unit-variance output
    err = float(np.abs(got_ln.astype(np.float64) - want_ln).max())
    print("LayerNorm max-abs vs CPU %.3g" % err)
    assert err <= 1e-3, err


@pytest.mark.parametrize("c,k,h,w", [
    (32, 64, 16, 40),    # level-0 out-projection + residual, then the RCAB LayerNorm
    (64, 128, 16, 40),   # K 128 (split reduction): one 64-wide wave
    (64, 64, 256, 256),  # K 64, 1024 pixel tiles: two 32-wide waves per pixel tile
    (32, 64, 3, 44),     # 132 pixels: a partial tile
])
@pytest.mark.parametrize("order", ["plan", "free"])
def test_layernorm_of_the_residual_sum_in_the_epilogue(gpu_ok, monkeypatch, order, c, k, h, w):
    """Conv1x1 k->c -> Add -> ChanLn, the raw sum also read later (kept): the
    streaming launch stores the sum and its LayerNorm. Bitwise the unfused
    pass under MAXIM_PLAN_ORDER=1, to rounding in the default order; the CPU
    path to the GEMM bar."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    set_order(monkeypatch, order)
    rng = np.random.default_rng(c + k + h * w)
    hw = h * w
    X, R, T, Y, LN, Z = range(6)
    bufs = [(k, h, w), (c, h, w), (c, h, w), (c, h, w), (c, h, w), (c, h, w)]
    wt = he(rng, (c, k), k)
    b = (rng.standard_normal(c) * 0.1).astype(np.float32)
    g2 = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(c)).astype(np.float32)
    n = c * hw
    ops = [P.make_op(P.CONV1X1, dst=T, src=X, w=0, bias=1, c_in=k, c_out=c, h=h, wd=w),
           P.make_op(P.ADD, dst=Y, src=T, src2=R, n=n),
           P.make_op(P.CHAN_LN, dst=LN, src=Y, scale=2, bias=3, c=c, hw=hw),
           P.make_op(P.ADD, dst=Z, src=LN, src2=Y, n=n)]
    cp = P.CustomPlan(bufs, ops, [wt, b, g2, b2], input=X, output=Z)
    inputs = {X: rng.standard_normal(bufs[X]).astype(np.float32), R: rng.standard_normal(bufs[R]).astype(np.float32)}
    got, steps = run_plan(cp, inputs, Z)
    print("steps", steps)
    assert any(fam(s[2]).endswith("_f_lo") for s in steps), steps
    gpu = H.Gpu(cp)
    for bb, v in inputs.items():
        gpu.write_buf(bb, v)
    gpu.set_fusion(False)
    gpu.run_ops(0, len(ops))
    plain = gpu.read_buf(Z).reshape(bufs[Z])
    gpu.close()
    agree(got, plain, order, 1e-5 * (1 + float(np.abs(plain).max())), "passes")
    want = oracle_plan(cp, inputs, Z)
    err = float(np.abs(got.astype(np.float64) - want).max())
    print("max-abs vs CPU %.3g" % err)
    assert err <= 1e-3, err


@pytest.mark.parametrize("c,k,h,w", [
    (32, 48, 16, 40),    # one 32-wide wave per band
    (64, 96, 128, 256),  # two waves of a block per band (2048 pixel tiles)
    (64, 128, 8, 36),    # split reduction: one 64-wide wave per band
])
@pytest.mark.parametrize("order", ["plan", "free"])
def test_layernorm_statistics_from_the_producer(gpu_ok, monkeypatch, order, c, k, h, w):
    """Conv1x1 k->2c, then each half LayerNormed into its own 1x1 conv (the
    split-head gMLP's two branches) after an unrelated op: the first conv's
    epilogue writes both halves' statistics and the folded GEMMs read them
    (no statistics pass). Bitwise the unfused pass under MAXIM_PLAN_ORDER=1,
    to rounding in the default order; the CPU path to the GEMM bar; a run of
    ops that starts after the producer runs the statistics pass itself
    (bitwise the unfused pass in either order)."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    set_order(monkeypatch, order)
    rng = np.random.default_rng(c * 7 + k + h * w)
    hw = h * w
    X, Y, U, V, UN, VN, A, B, Z1, Z2 = range(10)
    bufs = [(k, h, w), (2 * c, h, w), (c, h, w), (c, h, w), (c, h, w), (c, h, w),
            (c, h, w), (c, h, w), (c, h, w), (c, h, w)]
    views = {U: (Y, 0), V: (Y, c * hw)}
    wts = [he(rng, (2 * c, k), k), (rng.standard_normal(2 * c) * 0.1).astype(np.float32),
           he(rng, (c, c), c), (rng.standard_normal(c) * 0.1).astype(np.float32),
           (1 + 0.1 * rng.standard_normal(c)).astype(np.float32), (0.1 * rng.standard_normal(c)).astype(np.float32),
           (1 + 0.1 * rng.standard_normal(c)).astype(np.float32), (0.1 * rng.standard_normal(c)).astype(np.float32)]
    ops = [P.make_op(P.CONV1X1, dst=Y, src=X, w=0, bias=1, c_in=k, c_out=2 * c, h=h, wd=w),
           P.make_op(P.ADD, dst=A, src=U, src2=V, n=c * hw),          # another reader in between
           P.make_op(P.CHAN_LN, dst=UN, src=U, scale=4, bias=5, c=c, hw=hw),
           P.make_op(P.CONV1X1, dst=Z1, src=UN, w=2, bias=3, c_in=c, c_out=c, h=h, wd=w),
           P.make_op(P.CHAN_LN, dst=VN, src=V, scale=6, bias=7, c=c, hw=hw),
           P.make_op(P.CONV1X1, dst=Z2, src=VN, w=2, bias=3, c_in=c, c_out=c, h=h, wd=w),
           P.make_op(P.ADD, dst=B, src=Z1, src2=Z2, n=c * hw)]
    cp = P.CustomPlan(bufs, ops, wts, input=X, output=B, views=views)
    x = rng.standard_normal(bufs[X]).astype(np.float32)
    gpu = H.Gpu(cp)
    gpu.write_buf(X, x)
    gpu.run_ops(0, len(ops))
    steps = gpu.steps()
    kernels = gpu.launches()
    got = gpu.read_buf(B).reshape(bufs[B])
    print("steps", steps)
    print("launches", kernels)
    assert fam(steps[0][2]).endswith("_f_lo"), steps
    assert not any(kn.startswith("mx_chan_ln") for _, kn in kernels), kernels
    # a run starting after the producer: the statistics pass runs itself
    y_full = gpu.read_buf(Y)
    gpu.poison()
    gpu.write_buf(Y, y_full)
    gpu.run_ops(2, len(ops))
    part = gpu.read_buf(B).reshape(bufs[B])
    gpu.set_fusion(False)
    gpu.write_buf(X, x)
    gpu.run_ops(0, len(ops))
    plain = gpu.read_buf(B).reshape(bufs[B])
    gpu.close()
    agree(got, plain, order, 1e-5 * (1 + float(np.abs(plain).max())), "passes")
    assert np.array_equal(part.view(np.uint32), plain.view(np.uint32)), "the partial run differs"
    want = oracle_plan(cp, {X: x}, B)
    err = float(np.abs(got.astype(np.float64) - want).max())
    print("max-abs vs CPU %.3g (max|cpu| %.3g)" % (err, float(np.abs(want).max())))
    assert err <= 1e-3, err


@pytest.mark.parametrize("c,h,w,second", [
    (32, 16, 40, True),    # the RCAB output, then a block's long skip: one pass
    (64, 9, 20, False),    # ChanScale -> Add only
    (16, 5, 7, True),      # 35 pixels: the scalar kernel
])
def test_channel_scale_with_residual_adds(gpu_ok, c, h, w, second):
    """ChanScale -> Add [-> Add] (src/exec_cpu.rs chan_scale and add): one
    pass that scales, adds the residual and then the second operand in the
    unfused order; bit-exact against the CPU path and the unfused pass."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    rng = np.random.default_rng(c * 31 + h * w)
    hw = h * w
    X, S, T, R, Y, R2, Z = range(7)
    bufs = [(c, h, w), (c, 1, 1), (c, h, w), (c, h, w), (c, h, w), (c, h, w), (c, h, w)]
    ops = [P.make_op(P.CHAN_SCALE, dst=T, src=X, src2=S, c=c, hw=hw),
           P.make_op(P.ADD, dst=Y, src=R, src2=T, n=c * hw)]
    if second:
        ops.append(P.make_op(P.ADD, dst=Z, src=Y, src2=R2, n=c * hw))
    out = Z if second else Y
    cp = P.CustomPlan(bufs, ops, [], input=X, output=out)
    inputs = {X: rng.standard_normal(bufs[X]).astype(np.float32),
              S: rng.standard_normal(bufs[S]).astype(np.float32),
              R: rng.standard_normal(bufs[R]).astype(np.float32),
              R2: rng.standard_normal(bufs[R2]).astype(np.float32)}
    got, steps = run_plan(cp, inputs, out)
    print("steps", steps)
    assert len(steps) == 1 and steps[0][2].startswith("mx_chan_scale_add"), steps
    want = oracle_plan(cp, inputs, out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("c,h,w", [
    (64, 16, 40),     # whole tiles
    (128, 14, 20),    # 280 pixels: a partial last tile
    (32, 9, 20),
])
def test_layernorm_statistics_from_the_channel_scale(gpu_ok, c, h, w):
    """ChanScale -> Add -> Add (an RCAB's output plus a block's skip), then
    the sum LayerNormed into a 1x1 conv after an unrelated reader: the
    scale-add pass writes the sum's statistics and the folded GEMM reads
    them (no statistics pass). Bitwise the unfused pass, also for a run of
    ops that starts after the producer; the CPU path to the GEMM bar."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    rng = np.random.default_rng(c * 13 + h * w)
    hw = h * w
    X, S, T, R, Y, R2, Z, A, ZN, O, OUT = range(11)
    bufs = [(c, h, w), (c, 1, 1), (c, h, w), (c, h, w), (c, h, w), (c, h, w), (c, h, w), (c, h, w),
            (c, h, w), (c, h, w), (c, h, w)]
    wts = [he(rng, (c, c), c), (rng.standard_normal(c) * 0.1).astype(np.float32),
           (1 + 0.1 * rng.standard_normal(c)).astype(np.float32), (0.1 * rng.standard_normal(c)).astype(np.float32)]
    ops = [P.make_op(P.CHAN_SCALE, dst=T, src=X, src2=S, c=c, hw=hw),
           P.make_op(P.ADD, dst=Y, src=R, src2=T, n=c * hw),
           P.make_op(P.ADD, dst=Z, src=Y, src2=R2, n=c * hw),
           P.make_op(P.ADD, dst=A, src=Z, src2=R, n=c * hw),          # another reader in between
           P.make_op(P.CHAN_LN, dst=ZN, src=Z, scale=2, bias=3, c=c, hw=hw),
           P.make_op(P.CONV1X1, dst=O, src=ZN, w=0, bias=1, c_in=c, c_out=c, h=h, wd=w),
           P.make_op(P.ADD, dst=OUT, src=O, src2=A, n=c * hw)]
    cp = P.CustomPlan(bufs, ops, wts, input=X, output=OUT)
    inputs = {X: rng.standard_normal(bufs[X]).astype(np.float32),
              S: rng.standard_normal(bufs[S]).astype(np.float32),
              R: rng.standard_normal(bufs[R]).astype(np.float32),
              R2: rng.standard_normal(bufs[R2]).astype(np.float32)}
    gpu = H.Gpu(cp)
    for b, v in inputs.items():
        gpu.write_buf(b, v)
    gpu.run_ops(0, len(ops))
    steps = gpu.steps()
    kernels = gpu.launches()
    got = gpu.read_buf(OUT).reshape(bufs[OUT])
    print("steps", steps)
    print("launches", kernels)
    assert steps[0][2].startswith("mx_chan_scale_add_stats_c%d" % c), steps
    assert not any(kn.startswith("mx_chan_ln") for _, kn in kernels), kernels
    # a run starting after the producer: the statistics pass runs itself
    z_full = gpu.read_buf(Z)
    a_full = gpu.read_buf(A)
    gpu.poison()
    gpu.write_buf(Z, z_full)
    gpu.write_buf(A, a_full)
    gpu.run_ops(4, len(ops))
    part = gpu.read_buf(OUT).reshape(bufs[OUT])
    gpu.set_fusion(False)
    for b, v in inputs.items():
        gpu.write_buf(b, v)
    gpu.run_ops(0, len(ops))
    plain = gpu.read_buf(OUT).reshape(bufs[OUT])
    gpu.close()
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32)), "fused and unfused passes differ"
    assert np.array_equal(part.view(np.uint32), plain.view(np.uint32)), "the partial run differs"
    want = oracle_plan(cp, inputs, OUT)
    err = float(np.abs(got.astype(np.float64) - want).max())
    print("max-abs vs CPU %.3g (max|cpu| %.3g)" % (err, float(np.abs(want).max())))
    assert err <= 1e-3, err
