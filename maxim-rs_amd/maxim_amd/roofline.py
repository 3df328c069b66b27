"""Algorithmic cost of each op, for roofline fractions.

FLOPs = 2 x multiply-adds of the op as defined (no padding or halo work).
Bytes = compulsory fp32 traffic: every input read once, the output written
once, the weights read once. A fused kernel is charged its fused op's bytes.
Peaks are MI355X's published dense figures.
"""

from . import plan as P

PEAK_FP32_MFMA = 157.3e12   # FLOP/s
PEAK_HBM = 8.0e12           # B/s
RIDGE = PEAK_FP32_MFMA / PEAK_HBM

GEMM_KINDS = {P.CONV1X1, P.CONV3X3, P.CONV4X4S2, P.CONVT2X2, P.GATE_MM}


def op_cost(op):
    """(flops, bytes) of one op."""
    k = op.kind
    f4 = 4
    if k in (P.ADD, P.MUL, P.GATE_APPLY):
        return op.n, 3 * f4 * op.n
    if k in (P.GELU, P.LRELU, P.SIGMOID, P.COPY):
        return 0, 2 * f4 * op.n
    if k == P.CHAN_LN:
        return 0, f4 * (2 * op.c * op.hw + 2 * op.c)
    if k == P.CHAN_MEAN:
        return 0, f4 * (op.c * op.hw + op.c)
    if k == P.CHAN_SCALE:
        return 0, f4 * (2 * op.c * op.hw + op.c)
    if k == P.CONV1X1:
        pl = op.h * op.wd
        b = op.c_out if op.bias >= 0 else 0
        return 2 * op.c_in * op.c_out * pl, f4 * (op.c_in * pl + op.c_out * pl + op.c_in * op.c_out + b)
    if k == P.CONV3X3:
        pl = op.h * op.wd
        b = op.c_out if op.bias >= 0 else 0
        return 2 * 9 * op.c_in * op.c_out * pl, f4 * (op.c_in * pl + op.c_out * pl + 9 * op.c_in * op.c_out + b)
    if k == P.CONV4X4S2:
        pl, opl = op.h * op.wd, op.oh * op.ow
        b = op.c_out if op.bias >= 0 else 0
        return 2 * 16 * op.c_in * op.c_out * opl, f4 * (op.c_in * pl + op.c_out * opl + 16 * op.c_in * op.c_out + b)
    if k == P.CONVT2X2:
        pl = op.h * op.wd
        b = op.c_out if op.bias >= 0 else 0
        return 2 * 4 * op.c_in * op.c_out * pl, f4 * (op.c_in * pl + 4 * op.c_out * pl + 4 * op.c_in * op.c_out + b)
    if k == P.GATE_MM:
        outer, inner = op.p[0], op.p[1]
        kk = outer if op.mode == 0 else inner
        b = kk if op.bias >= 0 else 0
        return 2 * op.c * outer * inner * kk, f4 * (2 * op.c * outer * inner + kk * kk + b)
    if k == P.BLOCK_PERM:
        return 0, 2 * f4 * op.c * op.h * op.wd
    if k == P.RESIZE:
        # the plan's `tmp` operand ([c][hin][wout]) is written once and read once
        return 0, f4 * (op.c * op.h * op.wd + 2 * op.c * op.h * op.ow + op.c * op.oh * op.ow)
    if k == P.DOWN_S:
        return 0, 2 * f4 * op.c * op.oh * op.ow
    raise ValueError(k)


def bound_s(op):
    """The op's roofline time: max(flops / peak, bytes / bandwidth)."""
    f, b = op_cost(op)
    return max(f / PEAK_FP32_MFMA, b / PEAK_HBM)


def plan_cost(plan):
    fl = by = t = 0.0
    for op in plan.ops:
        f, b = op_cost(op)
        fl += f
        by += b
        t += bound_s(op)
    return fl, by, t
