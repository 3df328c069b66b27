"""C5: MAXIM-3S at 4096x4096 (the largest benchmark configuration: a ~29 GiB arena
resident in HBM), checked through properties that do not need a full CPU
pass (about five CPU minutes at this size):

  - the fused program's output is finite and bitwise identical run to run;
  - a lockstep walk of the unfused per-op launches from the same input, in
    which one instance of every op kind - the one with the largest output -
    is checked against the CPU oracle on the device's own operands, at the
    per-op bars of the C4-sized walks (bit-exact for permutations, resize,
    LayerNorm and the elementwise ops; 1e-4 * max|cpu| for the GEMMs);
  - the walk's final image agrees with the fused program's within the
    north-star bar (max-abs 2e-3, PSNR >= 50 dB): every fusion, folding and
    layout decision at this size against plain per-op execution.
"""

import time

import numpy as np
import pytest

from conftest import buf, judge_op, op_sources, psnr, weights

pytestmark = pytest.mark.gpu

SIDE = 4096


def c5_image():
    rng = np.random.default_rng(55)
    img = rng.random((3, SIDE, SIDE), dtype=np.float32)
    img += rng.normal(0.0, 0.05, size=img.shape).astype(np.float32)
    return np.clip(img, 0.0, 1.0)


def test_c5_maxim_3s_4096(gpu_ok):
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    from oracle import oracle as O

    plan = P.Plan(weights("S-3"), SIDE, SIDE)
    assert len(plan.ops) == 2885
    img = c5_image()
    gpu = H.Gpu(plan)
    print("C5: arena %.1f GiB" % (plan.arena_len * 4 / 2**30), flush=True)
    t = time.perf_counter()
    out = gpu.run(img)
    print("C5 fused pass 1: %.2f s (first pass, weights uploading)" % (time.perf_counter() - t), flush=True)
    t = time.perf_counter()
    again = gpu.run(img)
    print("C5 fused pass 2: %.2f s" % (time.perf_counter() - t), flush=True)
    assert np.isfinite(out).all()
    assert np.array_equal(out.view(np.uint32), again.view(np.uint32)), "C5 passes differ"
    del again

    # One op of each kind, the one with the largest output (the first of equals).
    pick = {}
    for i, op in enumerate(plan.ops):
        n = plan.buf_len(op.dst)
        if op.kind not in pick or n > pick[op.kind][1]:
            pick[op.kind] = (i, n)
    check = {i for i, _ in pick.values()}

    arena = np.zeros(plan.arena_len, np.float32)  # pages are touched only where written
    gpu.begin(img)
    failures = []
    for i, op in enumerate(plan.ops):
        if i not in check:
            gpu.step_op(i)
            continue
        for s in op_sources(plan, op):
            buf(plan, arena, s)[:] = gpu.read_buf(s)
        gpu.step_op(i)
        t = time.perf_counter()
        O.step(plan, arena, i)
        ok, key, err = judge_op(plan, arena, op, gpu.read_buf(op.dst))
        print("C5 op %4d %-40s %-10s err %.3g (cpu %.1f s)%s"
              % (i, op.describe(), key, err, time.perf_counter() - t, "" if ok else "  FAIL"), flush=True)
        if not ok:
            failures.append("op %d %s: %.3g" % (i, op.describe(), err))
    walked = gpu.read_buf(plan.output).reshape(out.shape)
    gpu.close()
    assert not failures, "\n".join(failures)
    err = float(np.abs(walked.astype(np.float64) - out).max())
    p = psnr(walked, out)
    print("C5 fused program vs per-op walk: max-abs %.3g, PSNR %.1f dB" % (err, p), flush=True)
    assert err <= 2e-3 and p >= 50.0
