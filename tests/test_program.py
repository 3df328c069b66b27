"""The executor's program, checked on the CPU: which ops fuse into one launch,
and the device arena it lays out by fused steps (include/maxim_hip.h,
mxh_plan_program). No device is used.

The layout must keep every operand of a step apart (a fused kernel reads its
inputs and writes its output at once), keep each op's output off its own
inputs (the reference's tests/packing.rs:87-118 rule), never let two live
buffers share storage, and - the semantic check - running the CPU path on
the device layout must give bitwise the image it gives on the plan's layout.
"""

import ctypes as C

import numpy as np
import pytest

from conftest import buf, weights


def program(plan, repack=True):
    from maxim_amd import hip as H
    L = H._lib()
    f = L.mxh_plan_program
    f.restype = C.c_int
    U = C.POINTER(C.c_uint64)
    f.argtypes = [C.POINTER(type(plan.desc)), C.c_int, U, U, U, U, U, U]
    n = len(plan.ops)
    fused, alen, nsteps = C.c_uint64(), C.c_uint64(), C.c_uint64()
    offs = np.zeros(len(plan.bufs), np.uint64)
    first = np.zeros(n, np.uint64)
    last = np.zeros(n, np.uint64)
    rc = f(C.byref(plan.desc), int(repack), C.byref(fused), C.byref(alen),
           offs.ctypes.data_as(U), first.ctypes.data_as(U), last.ctypes.data_as(U), C.byref(nsteps))
    assert rc == 0, H.P.last_error() if hasattr(H, "P") else rc
    k = nsteps.value
    return fused.value, alen.value, offs, list(zip(first[:k].astype(int), last[:k].astype(int)))


def base_of(plan, repack=True):
    """The owner of every buffer's device storage (view bases, and elided
    copies' sources sharing their destination)."""
    from maxim_amd import hip as H
    L = H._lib()
    f = L.mxh_plan_storage
    f.restype = C.c_int
    f.argtypes = [C.POINTER(type(plan.desc)), C.c_int, C.POINTER(C.c_int64)]
    owner = np.zeros(len(plan.bufs), np.int64)
    assert f(C.byref(plan.desc), int(repack), owner.ctypes.data_as(C.POINTER(C.c_int64))) == 0
    return [int(x) for x in owner]


@pytest.mark.parametrize("variant,h,w", [("S-2", 64, 64), ("S-3", 448, 640)])
def test_device_layout_is_sound(variant, h, w):
    from maxim_amd import plan as P
    plan = P.Plan(weights(variant), h, w)
    fused, alen, offs, steps = program(plan)
    print("%s %dx%d: %d of %d ops fused away, device arena %.1f MiB (plan %.1f MiB)"
          % (variant, h, w, fused, len(plan.ops), alen * 4 / 2**20, plan.arena_bytes / 2**20))
    assert fused >= 0.2 * len(plan.ops)
    # the device layout packs by fused steps, but keeps the buffers of the
    # paired gMLP branches apart over their regions (both run side by side)
    assert alen <= 1.6 * plan.arena_len
    assert steps[0][0] == 0 and steps[-1][1] == len(plan.ops)
    base = base_of(plan)

    def rng(b):
        return int(offs[b]), int(offs[b]) + plan.buf_len(b)

    def ov(x, y):
        return x[0] < y[1] and y[0] < x[1]

    for a, b in steps:
        ids = sorted({x for k in range(a, b) for x in plan.operands(plan.ops[k])})
        for i, x in enumerate(ids):
            assert rng(x)[1] <= alen
            for y in ids[i + 1:]:
                if base[x] != base[y]:
                    assert not ov(rng(x), rng(y)), ("step", a, b, x, y)
    elided = 0
    for k, op in enumerate(plan.ops):
        ids = plan.operands(op)
        if op.kind == P.COPY and offs[op.src] == offs[op.dst]:
            # an elided copy: its source was laid out on its destination
            assert base[op.src] == base[op.dst], ("op", k)
            elided += 1
            continue
        for s in ids[1:]:
            assert not ov(rng(ids[0]), rng(s)), ("op", k)
    print("%d copies elided" % elided)
    # live owning buffers never share storage (step-level live ranges)
    step_of = np.zeros(len(plan.ops), int)
    for si, (a, b) in enumerate(steps):
        step_of[a:b] = si
    first, last = {}, {}
    for k, op in enumerate(plan.ops):
        for x in plan.operands(op):
            r = base[x]
            first.setdefault(r, step_of[k])
            last[r] = max(last.get(r, 0), step_of[k])
    roots = sorted(first)
    lo = np.array([int(offs[r]) for r in roots])
    hi = lo + np.array([plan.buf_len(r) for r in roots])
    f = np.array([first[r] for r in roots])
    l = np.array([last[r] for r in roots])
    for i in range(len(roots)):
        clash = (lo[i] < hi[i + 1:]) & (lo[i + 1:] < hi[i]) & (f[i] <= l[i + 1:]) & (f[i + 1:] <= l[i])
        assert not clash.any(), roots[i]


def test_the_cpu_path_on_the_device_layout_is_bitwise_the_same():
    """Run the CPU oracle on the executor's arena layout (the plan with its
    offsets replaced) and on the plan's own: the images agree to the bit."""
    from maxim_amd import plan as P
    from oracle import oracle as O
    plan = P.Plan(weights("S-2"), 64, 64)
    fused, alen, offs, steps = program(plan)
    img = np.random.default_rng(4).random((3, 64, 64), dtype=np.float32)
    a = np.zeros(plan.arena_len, np.float32)
    a[int(plan.offs[plan.input]):int(plan.offs[plan.input]) + img.size] = img.ravel()
    O.run(plan, a)
    want = buf(plan, a, plan.output).copy()
    dev_offs = (C.c_uint64 * len(offs))(*[int(x) for x in offs])
    d = type(plan.desc)()
    C.pointer(d)[0] = plan.desc
    d.offs = dev_offs
    d.arena_len = alen
    b = np.zeros(alen, np.float32)
    b[int(offs[plan.input]):int(offs[plan.input]) + img.size] = img.ravel()
    rc = O.lib().oracle_run(C.byref(d), b.ctypes.data, 0)
    assert rc == 0
    o = int(offs[plan.output])
    got = b[o:o + want.size]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_without_a_view_table_the_plan_layout_is_kept():
    from maxim_amd import plan as P
    plan = P.Plan(weights("S-2"), 64, 64)
    fused, alen, offs, steps = program(plan, repack=False)
    assert alen == plan.arena_len and np.array_equal(offs, plan.offs)
    assert fused > 0
