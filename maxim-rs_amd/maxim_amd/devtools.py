"""The reference's development tools over the HIP executor.

  verify_walk      the --verify-gpu lockstep walk (src/main.rs:672-730): both
                   backends step the plan op by op from the same input, and
                   every op's destination is compared (bar: max|d| <= 1e-3 *
                   max|cpu|, src/main.rs:709-712); the first failures are
                   reported with the op, its buffer label and the element.
  verify_program_walk
                   the same lockstep check over the FUSED program the timed
                   path runs (no counterpart in the reference, which launches
                   one kernel per op): step by step, each step given the CPU
                   path's exact inputs, every buffer the step leaves for a
                   later op compared.
  timeline_report  the --profile census (src/main.rs:526-656): device time
                   per op family, per op shape (the 12 most expensive and
                   every shape with 16 or more ops) and the five slowest ops,
                   from per-op events with fusion off, plus the fused
                   program's time per kernel.
  dump_named       the --dump activations (src/image.rs:250-269): every named
                   buffer of a `named` plan as `<name>.npy`, [c][h][w] float32.
  compare_dumps    tools/compare.py: two dump directories tensor by tensor,
                   max-abs, RMS and PSNR, RMS above `tol` (1e-4) a failure,
                   in stage/level order.

The CPU side of the walk is the caller's: `cpu_step(plan, arena, i)` runs op
i of the CPU path on a host arena (the reference's exec_cpu::step). This
package never computes on the host itself.

    python -m maxim_amd.devtools compare REF_DIR MINE_DIR [--tol 1e-4]
"""

import argparse
import collections
import os
import re
import sys

import numpy as np

from . import plan as P


def op_sources(plan, op):
    """The arena buffers an op reads (a resize's second operand is its
    intermediate plane, written by the op itself)."""
    return [op.src] if op.kind == P.RESIZE else plan.operands(op)[1:]


def _buf(plan, arena, b):
    o = int(plan.offs[b])
    return arena[o:o + plan.buf_len(b)]


def reference_judge(tol):
    """The reference's per-op bar: max|d| <= tol * max|cpu| over the op's
    destination (src/main.rs:705-712)."""

    def judge(plan, arena, op, got):
        want = _buf(plan, arena, op.dst)
        d = np.abs(got.astype(np.float64) - want)
        scale = max(float(np.abs(want).max()) if want.size else 0.0, 1e-6)
        at = int(d.argmax()) if d.size else 0
        mx = float(d[at]) if d.size else 0.0
        return mx <= tol * scale, P.OP_NAMES[op.kind], mx / scale, at

    return judge


def verify_walk(plan, image, cpu_step, judge=None, resync=False, tol=1e-3, max_report=20, out=None):
    """Step the plan on the device and on the CPU path in lockstep from
    `image`, comparing every op's destination.

    `judge(plan, cpu_arena, op, got)` returns (ok, key, relative error[,
    element]); the default is the reference's 1e-3 * max|cpu| bar. With
    `resync` the device first receives the CPU path's exact source buffers
    for every op, so each op is judged on identical inputs (an op's own
    error, not an accumulation). Returns a dict: ops, bad, worst (largest
    relative error), worst_by_key, first (the first failing op's record) and
    failures (the first `max_report` records)."""
    from . import hip as H
    judge = judge or reference_judge(tol)
    img = np.ascontiguousarray(image, np.float32)
    arena = np.zeros(plan.arena_len, np.float32)
    o = int(plan.offs[plan.input])
    arena[o:o + img.size] = img.ravel()
    gpu = H.Gpu(plan)
    try:
        gpu.begin(img)
        worst, by_key, failures, bad = 0.0, {}, [], 0
        for i, op in enumerate(plan.ops):
            if resync:
                for s in op_sources(plan, op):
                    gpu.write_buf(s, _buf(plan, arena, s))
            cpu_step(plan, arena, i)
            gpu.step_op(i)
            r = judge(plan, arena, op, gpu.read_buf(op.dst))
            ok, key, rel = r[0], r[1], r[2]
            worst = max(worst, rel)
            by_key[key] = max(by_key.get(key, 0.0), rel)
            if not ok:
                bad += 1
                rec = {"op": i, "describe": op.describe(), "buf": int(op.dst), "relative": rel,
                       "element": int(r[3]) if len(r) > 3 else None, "key": key}
                if len(failures) < max_report:
                    failures.append(rec)
                    if out:
                        out("op %d: %s #%d differs by %.4e relative (element %s)"
                            % (i, rec["describe"], rec["buf"], rel, rec["element"]))
        if out:
            out("verify: %d ops, %d disagree beyond the bar (worst %.3e relative)" % (len(plan.ops), bad, worst))
        return {"ops": len(plan.ops), "bad": bad, "worst": worst, "worst_by_key": by_key,
                "first": failures[0] if failures else None, "failures": failures}
    finally:
        gpu.close()


def verify_program_walk(plan, image, cpu_step, tol=1e-4, max_report=20, out=None):
    """The fused program (mxh_steps: fused launches, paired branches,
    folded LayerNorms and permutations, commuted resizes; the default
    arithmetic order, not MAXIM_PLAN_ORDER=1) stepped against the CPU path.

    Before each step the device receives the CPU path's exact values of
    every buffer the step's ops read from earlier ops (for a permutation the
    executor elides, whose readers take its source through a map, that
    source); the step runs as it runs in a pass (mxh_run_ops over its op
    range: a folded LayerNorm whose statistics an earlier step wrote gets
    its statistics pass first), the CPU path runs the step's ops, and every
    buffer the step writes that a later op reads, or the plan's output, is
    judged: max|d| <= tol * max|cpu|. Buffers inside a step are never
    materialised and an elided permutation's output is never written, so
    neither is compared. Returns a dict: steps, compared (buffers), bad,
    worst, worst_by_kernel (by the kernel naming each step), kernels (every
    kernel the program launches), failures (the first `max_report`)."""
    from . import hip as H
    img = np.ascontiguousarray(image, np.float32)
    arena = np.zeros(plan.arena_len, np.float32)
    o = int(plan.offs[plan.input])
    arena[o:o + img.size] = img.ravel()
    last_read = {}
    for i, op in enumerate(plan.ops):
        for s in op_sources(plan, op):
            last_read[s] = i
    gpu = H.Gpu(plan)
    try:
        gpu.begin(img)
        steps = gpu.steps()
        # the permutations no launch computes (elided: their readers take the
        # source through a map), alone or inside a step of paired launches
        covered = set()
        for (a0, b0), second in gpu.launch_spans():
            covered.update(range(a0, b0))
            if second is not None:
                covered.update(range(*second))
        elided = {op.dst: op.src for i, op in enumerate(plan.ops)
                  if op.kind == P.BLOCK_PERM and i not in covered}
        worst, by_kernel, failures, bad, compared = 0.0, {}, [], 0, 0
        for n, (a, b, kernel) in enumerate(steps):
            made = set()
            for i in range(a, b):
                for s in op_sources(plan, plan.ops[i]):
                    if s in made:
                        continue
                    while s in elided:
                        s = elided[s]
                    gpu.write_buf(s, _buf(plan, arena, s))
                made.add(plan.ops[i].dst)
            for i in range(a, b):
                cpu_step(plan, arena, i)
            gpu.run_ops(a, b)
            for d in sorted(made):
                if d in elided or not (last_read.get(d, -1) >= b or d == plan.output):
                    continue
                want = _buf(plan, arena, d)
                got = gpu.read_buf(d)
                diff = np.abs(got.astype(np.float64) - want)
                scale = max(float(np.abs(want).max()) if want.size else 0.0, 1e-6)
                at = int(diff.argmax()) if diff.size else 0
                rel = float(diff[at]) / scale if diff.size else 0.0
                if not np.isfinite(got).all():
                    rel = float("inf")
                compared += 1
                worst = max(worst, rel)
                key = kernel or "(no launch)"
                by_kernel[key] = max(by_kernel.get(key, 0.0), rel)
                if not rel <= tol:
                    bad += 1
                    rec = {"step": n, "ops": (a, b), "kernel": kernel, "buf": int(d), "relative": rel,
                           "element": at, "describe": plan.ops[b - 1].describe()}
                    if len(failures) < max_report:
                        failures.append(rec)
                        if out:
                            out("step %d (ops %d-%d, %s): #%d differs by %.4e relative (element %d)"
                                % (n, a, b - 1, kernel, d, rel, at))
        if out:
            out("program walk: %d steps, %d buffers compared, %d beyond the bar (worst %.3e relative)"
                % (len(steps), compared, bad, worst))
        return {"steps": len(steps), "compared": compared, "bad": bad, "worst": worst,
                "worst_by_kernel": by_kernel, "kernels": sorted({k for _, k in gpu.launches()}),
                "failures": failures}
    finally:
        gpu.close()


def timeline_report(plan, image, out=print):
    """The --profile census of one pass (src/main.rs:526-656): per-op device
    times (fusion off, an event pair per op) by family, by shape and the
    slowest five; then the fused program's launches by kernel (run_timed:
    each launch timed by its own dispatch events). Returns a dict: per_op
    (ms per op), total_ms (the timeline's total), families ({family: [ms,
    ops]}), slowest (the five op indices), kernels ({kernel: [ms,
    launches]}) and fused_total_ms (run_timed's total)."""
    from . import hip as H
    gpu = H.Gpu(plan)
    try:
        gpu.set_fusion(False)
        gpu.set_timeline(True)
        gpu.run(image)
        per_op, total = gpu.timeline()
        fams = collections.defaultdict(lambda: [0.0, 0])
        shapes = collections.defaultdict(lambda: [0.0, 0])
        for i, op in enumerate(plan.ops):
            d = op.describe()
            fams[d.split()[0]][0] += float(per_op[i])
            fams[d.split()[0]][1] += 1
            shapes[d][0] += float(per_op[i])
            shapes[d][1] += 1
        out("timeline: %.2f ms total, %d ops (one launch stream per op, fusion off)" % (total, len(plan.ops)))
        out("%-12s %7s %9s %10s  %s" % ("op", "count", "total ms", "ms/op", "share"))
        for k, (ms, n) in sorted(fams.items(), key=lambda kv: -kv[1][0]):
            out("%-12s %7d %9.2f %10.4f  %5.1f%%" % (k, n, ms, ms / n, 100 * ms / max(total, 1e-9)))
        rows = sorted(shapes.items(), key=lambda kv: -kv[1][0])
        out("by shape:")
        for k, (ms, n) in rows[:12]:
            out("  %9.2f ms %5dx  %s" % (ms, n, k))
        out("  -- every other shape with 16 or more ops (aggregate, per-op):")
        for k, (ms, n) in rows[12:]:
            if n >= 16:
                out("  %9.2f ms %5dx  %s   (%.4f ms/op)" % (ms, n, k, ms / n))
        out("slowest ops:")
        slowest = [int(i) for i in np.argsort(-per_op, kind="stable")[:5]]
        for i in slowest:
            out("  op %d %.3f ms  %s" % (i, float(per_op[i]), plan.ops[i].describe()))
        # the fused program, launch by launch
        gpu.set_timeline(False)
        gpu.set_fusion(True)
        _, fused_total = gpu.run_timed()
        kern = collections.defaultdict(lambda: [0.0, 0])
        for (st, k), ms in zip(gpu.launches(), gpu.launch_timeline()):
            kern[k][0] += float(ms)
            kern[k][1] += 1
        tot = sum(v[0] for v in kern.values())
        out("fused program: %.2f ms of kernel time, %d launches" % (tot, sum(v[1] for v in kern.values())))
        for k, (ms, n) in sorted(kern.items(), key=lambda kv: -kv[1][0])[:12]:
            out("  %-30s %5d x %8.1f us  %5.1f%%" % (k, n, 1e3 * ms / n, 100 * ms / max(tot, 1e-9)))
        return {"per_op": per_op, "total_ms": total, "families": {k: list(v) for k, v in fams.items()},
                "slowest": slowest, "kernels": {k: list(v) for k, v in kern.items()},
                "fused_total_ms": fused_total}
    finally:
        gpu.close()


def dump_name(name):
    return name.replace("/", "_")


def dump_named(gpu, plan, outdir):
    """Every named activation of a `named` plan (after a pass) as
    outdir/<name>.npy, [c][h][w] float32 (the reference's save_npy layout).
    Returns the file paths."""
    os.makedirs(outdir, exist_ok=True)
    paths = []
    for name, b in plan.dumps:
        a = gpu.read_buf(b).reshape(plan.bufs[b])
        p = os.path.join(outdir, dump_name(name) + ".npy")
        np.save(p, a.astype(np.float32, copy=False))
        paths.append(p)
    return paths


def _psnr(a, b):
    d = np.asarray(a, np.float64) - np.asarray(b, np.float64)
    mse = float((d * d).mean()) if d.size else 0.0
    return float("inf") if mse == 0 else 10.0 * np.log10(1.0 / mse)


def _order(name):
    """Stage, then the numeric parts of the name (tools/compare.py's key)."""
    k = []
    for p in name.split("_"):
        m = re.match(r"^(.*?)(\d+)$", p)
        k.append((m.group(1), int(m.group(2))) if m else (p, -1))
    return k


def compare_dumps(ref_dir, mine_dir, tol=1e-4, out=print, show_all=False):
    """Diff two dump directories tensor by tensor (names matched by file
    stem; a leading singleton axis dropped on either side). Returns (rows,
    failures): rows of (name, shape, max-abs, rms, psnr)."""
    ref = {f[:-4]: os.path.join(ref_dir, f) for f in os.listdir(ref_dir) if f.endswith(".npy")}
    mine = {f[:-4]: os.path.join(mine_dir, f) for f in os.listdir(mine_dir) if f.endswith(".npy")}
    common = sorted(set(ref) & set(mine), key=_order)
    if not common:
        raise ValueError("compare: no names in common (ref has %d, mine has %d)" % (len(ref), len(mine)))
    out("%-40s %16s %12s %10s %8s" % ("tensor", "shape", "max abs", "rms", "psnr"))
    rows, failures = [], 0
    for name in common:
        a = np.load(ref[name]).squeeze()
        b = np.load(mine[name]).squeeze()
        if a.shape != b.shape:
            out("%-40s SHAPE %s vs %s" % (name, a.shape, b.shape))
            failures += 1
            rows.append((name, None, float("inf"), float("inf"), 0.0))
            continue
        d = a.astype(np.float64) - b
        mx = float(np.abs(d).max()) if d.size else 0.0
        rms = float(np.sqrt((d * d).mean())) if d.size else 0.0
        p = _psnr(a, b)
        bad = rms > tol
        failures += bad
        rows.append((name, a.shape, mx, rms, p))
        if bad or show_all:
            out("%-40s %16s %12.3e %10.3e %8.1f%s" % (name, "x".join(map(str, a.shape)), mx, rms, p,
                                                      "  FAIL" if bad else ""))
    out("compare: %d tensors, %d above RMS %.0e" % (len(common), failures, tol))
    return rows, failures


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m maxim_amd.devtools")
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("compare", help="diff two .npy dump directories (tools/compare.py)")
    c.add_argument("ref")
    c.add_argument("mine")
    c.add_argument("--tol", type=float, default=1e-4)
    c.add_argument("--all", action="store_true")
    args = ap.parse_args(argv)
    if args.cmd == "compare":
        _, failures = compare_dumps(args.ref, args.mine, args.tol, show_all=args.all)
        return 1 if failures else 0
    return 2


if __name__ == "__main__":
    sys.exit(main())
