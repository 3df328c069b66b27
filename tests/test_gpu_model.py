"""End-to-end parity of the HIP executor with the CPU oracle on whole MAXIM
passes (benchmark configurations C1 and C4), plus the properties the reference checks
for its own GPU path: poison-filled arenas give the same bytes
(src/exec_gpu.rs:313-340) and a pass is deterministic run to run.

Bar: final image within max-abs 2e-3 and PSNR >= 50
dB of the CPU path, compared on the UNCLAMPED output as well as the clamped one.
"""

import numpy as np
import pytest

from conftest import buf, psnr, run_oracle, smooth_image, weights

pytestmark = pytest.mark.gpu


def compare(plan, img, label, tol=2e-3):
    from maxim_amd import hip as H
    gpu = H.Gpu(plan)
    out = gpu.run(img)
    arena = run_oracle(plan, img)
    ref = buf(plan, arena, plan.output).reshape(out.shape)
    err = float(np.abs(out.astype(np.float64) - ref).max())
    clamped = float(np.abs(np.clip(out, 0, 1) - np.clip(ref, 0, 1)).max())
    p = psnr(out, ref)
    print("%s: unclamped max-abs %.3g, clamped %.3g, PSNR %.1f dB, output range [%.3f, %.3f]"
          % (label, err, clamped, p, float(ref.min()), float(ref.max())), flush=True)
    assert np.isfinite(out).all()
    assert err <= tol, "%s: max-abs %.3g > %.3g" % (label, err, tol)
    assert p >= 50.0, "%s: PSNR %.1f dB < 50" % (label, p)
    return gpu, out


def test_c1_maxim_2s_256(gpu_ok):
    """C1: MAXIM-2S, seeded weights, one 256x256 RGB input U[0,1)."""
    from maxim_amd import plan as P
    plan = P.Plan(weights("S-2"), 256, 256)
    assert len(plan.ops) == 1840
    img = np.random.default_rng(11).random((3, 256, 256), dtype=np.float32)
    compare(plan, img, "C1 S-2 256x256")


def test_c4_maxim_3s_600x400(gpu_ok):
    """C4: MAXIM-3S, a 600x400 image (smooth pattern + N(0, 0.1), clipped),
    reflect-padded to 640x448 by the reference pipeline, cropped back."""
    from maxim_amd import plan as P
    raw = smooth_image(400, 600, seed=4)
    pad = P.preprocess(raw, 64)
    assert pad.img.shape == (3, 448, 640)
    plan = P.Plan(weights("S-3"), 448, 640)
    assert len(plan.ops) == 2885
    gpu, out = compare(plan, pad.img, "C4 S-3 640x448")
    crop = P.crop_out(out, pad)
    assert crop.shape == (3, 400, 600)
    # The timed path (bench.py): replays of the captured graph are bitwise the
    # eager fused pass just checked against the CPU path, replay after replay.
    out = out.copy()
    gpu.set_graph(True)
    for rep in range(2):
        got = gpu.run(pad.img)
        assert np.array_equal(got.view(np.uint32), out.view(np.uint32)), rep


def test_poison_and_determinism(gpu_ok):
    """A poisoned arena (0xCD everywhere) gives the same bytes as a clean one,
    and two passes are bitwise identical: nothing reads before it writes."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    plan = P.Plan(weights("S-2"), 128, 128)
    img = smooth_image(128, 128, seed=9)
    gpu = H.Gpu(plan)
    a = gpu.run(img)
    gpu.poison()
    b = gpu.run(img)
    c = gpu.run(img)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(b.view(np.uint32), c.view(np.uint32))


def test_he_normal_unscaled_relative(gpu_ok):
    """Pure He-normal weights: outputs reach ~1e7, so the bar is relative
    (the reference's own per-op bar, 1e-3 * max|cpu|)."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    plan = P.Plan(weights("S-2", gain=1.0, bias_std=0.0, ln_std=0.0), 128, 128)
    img = np.random.default_rng(2).random((3, 128, 128), dtype=np.float32)
    out = H.Gpu(plan).run(img)
    ref = buf(plan, run_oracle(plan, img), plan.output).reshape(out.shape)
    rel = float(np.abs(out.astype(np.float64) - ref).max() / np.abs(ref).max())
    print("unscaled He-normal: max|cpu| %.3g, relative error %.3g" % (float(np.abs(ref).max()), rel))
    assert rel <= 1e-3


def test_timeline_and_counters(gpu_ok):
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    plan = P.Plan(weights("S-2"), 64, 64)
    gpu = H.Gpu(plan)
    gpu.set_fusion(False)
    gpu.set_timeline(True)
    gpu.run(smooth_image(64, 64))
    per, total = gpu.timeline()
    assert per.shape == (1840,) and total > 0 and abs(per.sum() - total) < 1e-3 * total + 1e-3
    assert gpu.ops_launched == 1840
    assert gpu.kernels_launched >= 1840
    assert gpu.arena_bytes <= 1.6 * plan.arena_bytes
    gpu.set_fusion(True)
    steps = gpu.steps()
    assert steps[0][0] == 0 and steps[-1][1] == 1840
    assert all(a[1] == b[0] for a, b in zip(steps, steps[1:]))
    # fused_ops counts the ops that launch nothing of their own: those folded
    # into another op's step, and elided copies (a step with no kernel); a
    # step that pairs two branches' launches stands for several such steps
    empty = sum(1 for _, _, k in steps if not k)
    assert len(steps) - empty <= 1840 - gpu.fused_ops
    gpu.run(smooth_image(64, 64))
    per, total = gpu.timeline()
    assert per.shape == (len(steps),)
    # per-launch events: every launch names its step, and a step's time is
    # the sum of its launches'
    per, total = gpu.run_timed()
    launches = gpu.launches()
    ms = gpu.launch_timeline()
    assert len(launches) == len(ms) and all(0 <= st < len(steps) for st, _ in launches)
    assert [st for st, _ in launches] == sorted(st for st, _ in launches)
    sums = np.zeros(len(steps))
    for (st, _), t in zip(launches, ms):
        sums[st] += t
    assert np.allclose(sums, per, rtol=1e-5, atol=1e-6) and abs(ms.sum() - total) < 1e-3 * total + 1e-3


@pytest.mark.parametrize("variant,side", [("S-2", 128), ("S-3", 64), ("S-3", 448)])
def test_fusion_is_bitwise_transparent(gpu_ok, variant, side, monkeypatch):
    """The fused program applies each reader in its producer's epilogue with the
    same float operations, so fused and unfused passes agree to the bit (448:
    planes large enough for many CALayer mean partials, tens per channel).
    The one rule that reorders arithmetic (UpSampleRatio's resize and conv
    commuted, tests/test_gpu_commute.py) is switched off for the bitwise
    check, and with it on the passes agree to rounding."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    plan = P.Plan(weights(variant), side, side)
    img = smooth_image(side, side, seed=12)
    gpu = H.Gpu(plan)
    c = gpu.run(img).copy()
    gpu.close()
    monkeypatch.setenv("MAXIM_PLAN_ORDER", "1")
    gpu = H.Gpu(plan)
    gpu.set_fusion(False)
    a = gpu.run(img).copy()
    gpu.set_fusion(True)
    b = gpu.run(img)
    print("%s %d: %d of %d ops fused away; commuted pass vs op by op: max-abs %.3g"
          % (variant, side, gpu.fused_ops, len(plan.ops), float(np.abs(c.astype(np.float64) - a).max())))
    assert gpu.fused_ops > 300
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert float(np.abs(c.astype(np.float64) - a).max()) <= 2e-5


def test_graph_replays_match_eager(gpu_ok):
    """The captured graph launches the same kernels in the same order: every
    replay is bitwise the eager pass, with eager passes on other inputs in
    between the replays."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    plan = P.Plan(weights("S-2"), 128, 128)
    gpu = H.Gpu(plan)
    imgs = [smooth_image(128, 128, seed=s) for s in range(3)]
    eager = [gpu.run(im).copy() for im in imgs]
    for rep in range(4):
        k = rep % 3
        gpu.set_graph(True)
        got = gpu.run(imgs[k])
        gpu.set_graph(False)
        other = gpu.run(imgs[(k + 1) % 3])
        assert np.array_equal(got.view(np.uint32), eager[k].view(np.uint32)), rep
        assert np.array_equal(other.view(np.uint32), eager[(k + 1) % 3].view(np.uint32)), rep


def test_runs_of_ops_that_cut_fused_steps(gpu_ok, monkeypatch):
    """A pass run as contiguous runs of ops (mxh_run_ops), with every cut
    inside a fused step - among them steps that read an elided forward
    permutation's output, which then has to be restored - gives the full
    pass's bits (a cut step runs its ops in the plan's order, so the rule
    that commutes UpSampleRatio's resize and conv is off here)."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    monkeypatch.setenv("MAXIM_PLAN_ORDER", "1")
    plan = P.Plan(weights("S-3"), 64, 64)
    img = smooth_image(64, 64, seed=13)
    gpu = H.Gpu(plan)
    full = gpu.run(img).copy()
    steps = gpu.steps()
    perm_steps = {a for a, b, k in steps if b == a + 1 and not k and plan.ops[a].kind == P.BLOCK_PERM}
    multi = [(a, b) for a, b, k in steps if b - a >= 2]
    # cut inside every 7th multi-op step, and inside every step right after an elided permutation
    after_perm = [(a, b) for (a, b) in multi if any(q < a and q + 40 > a for q in perm_steps)]
    cuts = sorted({(a + b) // 2 for (a, b) in multi[::7] + after_perm[::3]})
    print("%d steps, %d elided permutations, %d cuts" % (len(steps), len(perm_steps), len(cuts)), flush=True)
    assert perm_steps and len(cuts) > 20
    gpu.begin(img)
    edges = [0] + cuts + [len(plan.ops)]
    for a, b in zip(edges, edges[1:]):
        gpu.run_ops(a, b)
    got = gpu.read_buf(plan.output).reshape(full.shape)
    assert np.array_equal(got.view(np.uint32), full.view(np.uint32))


def test_gmlp_branches_share_launches(gpu_ok):
    """At C4 the grid and block branches of the multi-axis gMLP blocks below
    full resolution run their in- and out-projections as paired launches
    (one grid for both): each paired launch names two disjoint op ranges
    inside its step, with the same GEMM (the ops fused around it may differ:
    one branch's output permutation folded into the stores, the other's
    launched apart) or the same LayerNorm, and the pass still equals the
    unpaired one to the bit (the paired steps' ops run in another order only
    where nothing they touch overlaps)."""
    import os
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    plan = P.Plan(weights("S-3"), 448, 640)
    img = smooth_image(448, 640, seed=21)
    gpu = H.Gpu(plan)
    got = gpu.run(img).copy()
    steps = gpu.steps()
    pairs = 0
    for (st, k), (r0, r1) in zip(gpu.launches(), gpu.launch_spans()):
        a, b, _ = steps[st]
        assert a <= r0[0] < r0[1] <= b
        if r1 is None:
            assert not k.endswith("_x2"), k
            continue
        pairs += 1
        assert k.endswith("_x2") and a <= r1[0] < r1[1] <= b and (r0[1] <= r1[0] or r1[1] <= r0[0])
        gemm = lambda r: [(op.kind, op.c_in, op.c_out, op.h * op.wd) for op in plan.ops[r[0]:r[1]]
                          if op.kind in (P.CONV1X1, P.GATE_MM)][:1]
        lns = lambda r: [(op.kind, op.c, op.hw) for op in plan.ops[r[0]:r[1]]]
        if k.startswith("mx_chan_ln"):
            assert lns(r0) == lns(r1) and [t[0] for t in lns(r0)] == [P.CHAN_LN], (k, r0, r1)
        else:
            assert gemm(r0) == gemm(r1) and gemm(r0), (k, r0, r1)
    gpu.close()
    print("%d paired launches" % pairs)
    assert pairs >= 40
    os.environ["MAXIM_NO_PAIR"] = "1"
    try:
        gpu = H.Gpu(plan)
        assert not any(k.endswith("_x2") for _, k in gpu.launches())
        ref = gpu.run(img)
        gpu.close()
    finally:
        del os.environ["MAXIM_NO_PAIR"]
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("variant,h,w,n,graph", [("S-2", 128, 192, 5, False), ("S-3", 448, 640, 3, True)])
def test_run_batch_equals_run_per_image(gpu_ok, variant, h, w, n, graph):
    """mxh_run_batch (pinned staging in two slots, the host's copies
    overlapped with the passes): each image's output is mxh_run's to the
    bit, for an odd count (the two staging slots alternate unevenly), with
    eager launches and with graph replays; an empty list does nothing, and a
    second batch on the same executor reuses the staging."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    plan = P.Plan(weights(variant), h, w)
    imgs = [smooth_image(h, w, seed=30 + k) for k in range(n)]
    gpu = H.Gpu(plan)
    gpu.set_graph(graph)
    want = [gpu.run(im).copy() for im in imgs]
    print("%s %dx%d: %d images, graph %s" % (variant, w, h, n, graph), flush=True)
    assert gpu.run_batch([]) == []
    for rep in range(2):
        got = gpu.run_batch(imgs if rep == 0 else imgs[::-1])
        for k, g in enumerate(got):
            ref = want[k] if rep == 0 else want[n - 1 - k]
            assert np.array_equal(g.view(np.uint32), ref.view(np.uint32)), (rep, k)
    gpu.close()
