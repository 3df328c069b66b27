"""The --profile census (src/main.rs:526-656; the per-op timeline of
src/exec_gpu.rs:231-265) through maxim_amd.devtools.timeline_report: a
timeline pass with fusion off (one event pair per op), then the fused
program timed launch by launch. Checked for internal consistency on MAXIM-2S
64x64: the families add up to the timeline's total and cover every op once,
the slowest five are the five largest per-op times and name real ops, and
the fused-kernel table adds up to run_timed's total over every launch."""

import numpy as np
import pytest

from conftest import weights

pytestmark = pytest.mark.gpu


def test_timeline_report_census(gpu_ok):
    from maxim_amd import devtools as D
    from maxim_amd import hip as H
    from maxim_amd import plan as P
    plan = P.Plan(weights("S-2"), 64, 64)
    img = np.random.default_rng(3).random(plan.shape, dtype=np.float32)
    lines = []
    print("profile: S-2 64x64 census", flush=True)
    rep = D.timeline_report(plan, img, out=lines.append)
    text = "\n".join(lines)
    print(text)
    n = len(plan.ops)
    per_op = rep["per_op"]
    # the timeline pass ran with fusion off: one time per op, every op launched
    assert len(per_op) == n and (per_op > 0).sum() >= 0.9 * n
    assert "fusion off" in lines[0] and "%d ops" % n in lines[0]
    # families: every op counted once, totals add up to the timeline's total
    fam = rep["families"]
    assert sum(c for _, c in fam.values()) == n
    assert abs(sum(ms for ms, _ in fam.values()) - rep["total_ms"]) <= 1e-3 * rep["total_ms"]
    assert abs(float(per_op.astype(np.float64).sum()) - rep["total_ms"]) <= 1e-3 * rep["total_ms"]
    kinds = {op.describe().split()[0] for op in plan.ops}
    assert set(fam) == kinds
    # the slowest five: the largest per-op times, each line naming its op
    top = rep["slowest"]
    assert len(top) == 5 and len(set(top)) == 5 and all(0 <= i < n for i in top)
    assert np.isclose(per_op[top[0]], per_op.max())
    assert min(per_op[i] for i in top) >= np.sort(per_op)[-5]
    at = lines.index("slowest ops:")
    for k, i in enumerate(top):
        assert lines[at + 1 + k].startswith("  op %d " % i) and plan.ops[i].describe() in lines[at + 1 + k]
    # the fused program: its kernel table adds up to run_timed's total, over
    # as many launches as the fused program has
    kern = rep["kernels"]
    assert abs(sum(ms for ms, _ in kern.values()) - rep["fused_total_ms"]) <= 1e-3 * rep["fused_total_ms"]
    g = H.Gpu(plan)
    try:
        g.run(img)
        nl = len(g.launches())
    finally:
        g.close()
    assert sum(c for _, c in kern.values()) == nl
    assert all(k.startswith("mx_") for k in kern)
    assert "fused program: %.2f ms" % sum(ms for ms, _ in kern.values()) in text
