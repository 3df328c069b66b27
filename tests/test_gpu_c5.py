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


def _abs_max(x, chunk=1 << 25):
    m = 0.0
    for a in range(0, x.size, chunk):
        m = max(m, float(np.abs(x[a:a + chunk]).max()))
    return m


def test_c5_fused_steps_against_cpu(gpu_ok):
    """The fused program the C5 bench times, one step per kernel that names a
    step - its largest instance at this size, so the tile counts, 64-bit
    offsets and grids of the full configuration - run as in a pass on the
    device's own inputs to that step, against the CPU path's ops over the
    same inputs: every buffer the step hands on within 1e-4 * max|cpu| (an
    elided permutation's output, which fused steps read through a map from
    its source, is formed on the CPU side from that source)."""
    import re
    from conftest import _max_abs_diff
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    from oracle import oracle as O

    plan = P.Plan(weights("S-3"), SIDE, SIDE)
    img = c5_image()
    gpu = H.Gpu(plan)
    steps = gpu.steps()
    last_read = {}
    for i, op in enumerate(plan.ops):
        for s in op_sources(plan, op):
            last_read[s] = i
    elided = {plan.ops[a].dst: a for a, b, k in steps
              if not k and b == a + 1 and plan.ops[a].kind == P.BLOCK_PERM}

    def handed_on(a, b):
        out = []
        for i in range(a, b):
            d = plan.ops[i].dst
            if d not in elided and d not in out and (last_read.get(d, -1) >= b or d == plan.output):
                out.append(d)
        return out

    pick = {}
    for n, (a, b, k) in enumerate(steps):
        size = sum(plan.buf_len(d) for d in handed_on(a, b))
        if k and size and (k not in pick or size > pick[k][1]):
            pick[k] = (n, size)
    chosen = {n for n, _ in pick.values()}
    print("C5: %d steps, %d kernels checked" % (len(steps), len(chosen)), flush=True)

    arena = np.zeros(plan.arena_len, np.float32)  # pages are touched only where written
    gpu.begin(img)
    failures, worst = [], {}
    for n, (a, b, k) in enumerate(steps):
        if n in chosen:
            made = set()
            for i in range(a, b):
                for s in op_sources(plan, plan.ops[i]):
                    if s in made:
                        continue
                    if s in elided:
                        j = elided[s]
                        buf(plan, arena, plan.ops[j].src)[:] = gpu.read_buf(plan.ops[j].src)
                        O.step(plan, arena, j)
                    else:
                        buf(plan, arena, s)[:] = gpu.read_buf(s)
                made.add(plan.ops[i].dst)
        gpu.run_ops(a, b)
        if n not in chosen:
            continue
        t = time.perf_counter()
        for i in range(a, b):
            O.step(plan, arena, i)
        for d in handed_on(a, b):
            want = buf(plan, arena, d)
            got = gpu.read_buf(d)
            finite = all(np.isfinite(got[c:c + (1 << 25)]).all() for c in range(0, got.size, 1 << 25))
            rel = _max_abs_diff(got, want) / max(_abs_max(want), 1e-6) if finite else float("inf")
            del got
            fam = re.sub(r"_e\d+$", "", k)
            worst[fam] = max(worst.get(fam, 0.0), rel)
            ok = rel <= 1e-4
            print("C5 step %4d ops %4d-%4d %-32s #%d %.3g relative (cpu %.1f s)%s"
                  % (n, a, b - 1, k, d, rel, time.perf_counter() - t, "" if ok else "  FAIL"), flush=True)
            if not ok:
                failures.append("step %d (%s) buffer %d: %.3g" % (n, k, d, rel))
    gpu.close()
    print("C5 worst by kernel:", sorted(worst.items(), key=lambda kv: -kv[1])[:8], flush=True)
    assert not failures, "\n".join(failures)
