"""Benchmark: MAXIM-3S forward pass on one MI355X (configuration C4).

One step = one MAXIM-3S forward pass (2885 ops) over one 600x400 RGB image
reflect-padded to 640x448, with the image and the weights already resident
in HBM when the timed region starts. Prints ONE JSON line:

  value         images/s (whole job; one GPU), from K replays of the captured
                graph of the fused program
  ms_per_step   ms/image (K back-to-back replays over the wall clock);
                `passes` gives the median, min and max of >= 10 replays each
                timed by its own HIP events, `e2e` the pass with the input
                copied in and the output copied out (PCIe included; never
                `value`), one image at a time and as a serving loop
                (mxh_run_batch, the host's staging overlapped with the
                passes), `program_roofline` the fused program's own bound
                (each launch's max(FLOPs / 157.3 TFLOP/s, bytes / 8 TB/s),
                summed) and the pass's fraction of it
  roofline      the dominant kernel's achieved rate against its bound (fp32
                MFMA 157.3 TFLOP/s or HBM 8 TB/s): algorithmic FLOPs or bytes
                per launch over the average launch duration, from the HIP
                start/stop events each dispatch records on the executor's
                stream over K further (eager) passes; `traffic` = its measured
                HBM-side bytes per launch (profiles/hbm_traffic_c4.md);
                `frac_of_own_bound` the same launches against each one's own
                roofline min(P, AI x B)
  cpu_baseline  the CPU path (oracle/, a C restatement of the reference's
                src/exec_cpu.rs) timed on this host: the median of three full
                C4 passes on every host core the process may use, plus one
                single-thread MAXIM-2S 256x256 (C1) pass and a single-thread
                C2 layer (one split-head gMLP layer, c = 32, 256x256) for
                scaling
  c5            the 4096x4096 configuration (C5, a 28.7 GiB arena): ms/image
                over graph replays, the dominant kernel's rate there (its
                tensors are far larger than the 256 MB Infinity Cache, so the
                HBM figure is cache-free), the whole pass's effective rate
                and a per-kernel table (the memory-bound kernels and the
                GEMMs with the most time: rate and fraction of its peak)
  validation    the last timed replay's output against the first (eager)
                pass, bit for bit, and against the CPU path (max-abs, PSNR);
                the run fails if they disagree

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-c5] [--variant S-3]
"""

import argparse
import collections
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "maxim-rs_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

METRIC = "ms/image & images/s, MAXIM-3S 640x448 fp32; GEMM % of MFMA peak, HBM GB/s"
SEED = 1
GAIN = 0.3


def smooth_image(h, w, seed=0, noise=0.1):
    rng = np.random.default_rng(seed)
    y, x = np.mgrid[0:h, 0:w].astype(np.float64)
    img = np.empty((3, h, w))
    for c in range(3):
        f = rng.uniform(0.5, 3.0, size=(3, 2))
        ph = rng.uniform(0, 2 * np.pi, size=3)
        v = 0.5 + sum(0.1 * np.sin(2 * np.pi * (f[k, 0] * y / h + f[k, 1] * x / w) + ph[k]) for k in range(3))
        img[c] = v + rng.normal(0, noise, size=(h, w))
    return np.clip(img, 0, 1).astype(np.float32)


def family(kernel):
    """Group kernel entry points into the family a roofline is quoted for."""
    for pre in ("mx_gemm", "mx_pw", "mx_conv3x3", "mx_c3", "mx_conv4x4", "mx_chan_ln", "mx_block_perm",
                "mx_resize", "mx_chan_mean", "mx_ca", "mx_gemv"):
        if kernel.startswith(pre):
            return pre
    return kernel.rsplit("_", 1)[0] if kernel.endswith(("_v4", "_s")) else kernel


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--eager", action="store_true",
                    help="time eager launches of the fused program instead of graph replays "
                         "(the same kernels; for tracing tools)")
    ap.add_argument("--no-c5", action="store_true", help="skip the 4096x4096 leg")
    ap.add_argument("--cpu-threads", type=int, default=host_threads())
    ap.add_argument("--variant", default="S-3", choices=["S-1", "S-2", "S-3", "M-1", "M-2", "M-3"],
                    help="the model (default S-3, the configuration the metric is quoted on)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (a MAXIM pass is one image on one device; "
              "data-parallel serving is N independent processes). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from maxim_amd import plan as P
    from maxim_amd import hip as H
    from maxim_amd import roofline as R

    name = model_name(args.variant)
    w = P.Weights.synthetic(args.variant, seed=SEED, gain=GAIN, bias_std=0.02, ln_std=0.1)
    raw = smooth_image(400, 600, seed=4)
    pad = P.preprocess(raw, 64)
    _, ph, pw = pad.img.shape
    plan = P.Plan(w, ph, pw)
    n_ops = len(plan.ops)
    print("bench: %s %dx%d, %d ops, arena %.1f MiB" % (name, pw, ph, n_ops, plan.arena_bytes / 2**20),
          file=sys.stderr, flush=True)

    gpu = H.Gpu(plan)
    # PCIe-inclusive pass (input H2D, ops, output D2H), reported on stderr only.
    t0 = time.perf_counter()
    out = gpu.run(pad.img)
    e2e_first = time.perf_counter() - t0
    assert np.isfinite(out).all(), "non-finite output"
    n_ops_all = len(plan.ops)
    one_pass = (lambda: gpu.run_ops(0, n_ops_all)) if args.eager else gpu.run_graph
    for _ in range(args.warmup):
        one_pass()
    gpu.sync()

    # Timed region: K passes over the resident image, each one replay of the
    # captured graph of the fused program (the executor's serving path; with
    # --eager the same launches issued one by one), bracketed by device
    # synchronisation.
    gpu.sync()
    t_start = time.perf_counter()
    for _ in range(args.steps):
        one_pass()
    gpu.sync()
    wall = time.perf_counter() - t_start
    ms_per_step = wall * 1e3 / args.steps
    # The last timed pass's output: the replays must reproduce the first
    # (eager) pass bit for bit (a program that dropped work, or an input
    # overwritten between replays, would not).
    out_last = gpu.read_buf(plan.output).reshape(out.shape)
    same = bool(np.array_equal(out_last.view(np.uint32), out.view(np.uint32)))

    # Per-pass device times: >= 10 replays, each bracketed by its own events.
    passes = None
    if not args.eager:
        pm = gpu.time_graph(max(10, args.steps))
        passes = {"median_ms": float(np.median(pm)), "min_ms": float(pm.min()), "max_ms": float(pm.max()),
                  "n": int(pm.size), "timing": "HIP events around each graph replay"}
    # End to end: host image in, pass, host image out (PCIe included).
    gpu.set_graph(not args.eager)
    e2e = []
    for _ in range(5):
        t0 = time.perf_counter()
        o2 = gpu.run(pad.img)
        e2e.append(time.perf_counter() - t0)
    # A serving loop: images host to host through mxh_run_batch, the host's
    # staging overlapped with the passes.
    nb = 12
    ob = gpu.run_batch([pad.img] * 2)
    t0 = time.perf_counter()
    ob = gpu.run_batch([pad.img] * nb)
    batch_s = (time.perf_counter() - t0) / nb
    gpu.set_graph(False)
    same = same and bool(np.array_equal(o2.view(np.uint32), out.view(np.uint32)))
    same = same and all(bool(np.array_equal(b.view(np.uint32), out.view(np.uint32))) for b in ob)
    e2e_rec = {"first_pass_ms": e2e_first * 1e3, "median_ms": float(np.median(e2e)) * 1e3, "n": len(e2e),
               "what": "mxh_run: input H2D + the pass (%s) + output D2H, host wall clock"
                       % ("graph replay" if not args.eager else "eager launches"),
               "batch_ms_per_image": batch_s * 1e3, "batch_images": nb,
               "batch_what": "mxh_run_batch over %d images, host arrays in and out, the host's staging "
                             "(pinned) overlapped with the passes; host wall clock / images" % nb}

    # Attribution: K more passes of the same program launched eagerly, each
    # launch timed by the start/stop events its dispatch records on the
    # executor's stream. Each launch is charged its kernel's algorithmic cost
    # (launch_costs).
    steps = gpu.steps()
    launches = gpu.launches()
    cost = launch_costs(plan, steps, launches, R, gpu.launch_spans())
    per_kernel = collections.defaultdict(lambda: [0.0, 0, 0.0, 0.0, 0.0])  # ms, launches, flops, bytes, bound ms
    ev_tot = []
    for _ in range(args.steps):
        _, tot = gpu.run_timed()
        ev_tot.append(tot)
        ms = gpu.launch_timeline()
        for k, (st, kn) in enumerate(launches):
            f, by = cost[k]
            e = per_kernel[kn]
            e[0] += float(ms[k])
            e[1] += 1
            e[2] += f
            e[3] += by
            e[4] += launch_bound_ms(f, by, R)
    ev_ms = float(np.median(ev_tot))
    prog_bound_ms = sum(launch_bound_ms(f, by, R) for f, by in cost)

    # The dominant kernel by device time; its arithmetic intensity picks the
    # roofline axis.
    kern, (tms, nl, fl, by, _) = max(per_kernel.items(), key=lambda kv: kv[1][0])
    avg_s = tms / nl / 1e3
    ai = fl / by if by else 0.0
    if ai >= R.RIDGE:
        roof = {"bound": "mfma", "achieved": fl / nl / avg_s / 1e12, "peak": 157.3, "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": by / nl / avg_s / 1e9, "peak": 8000.0, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = traffic_per_launch(kern)
    roof["kernel"] = kern
    roof["avg_launch_us"] = avg_s * 1e6
    roof["launches_per_step"] = nl // args.steps
    roof["algorithmic_per_launch"] = {"gflop": fl / nl / 1e9, "mb": by / nl / 1e6}
    roof["frac_of_own_bound"] = per_kernel[kern][4] / tms

    fl_all, by_all, bound_s = R.plan_cost(plan)
    print("bench: %.3f ms/image (%s), %.3f ms event-timed eager pass, %d steps for %d ops; "
          "roofline sum of per-op bounds %.2f ms" % (ms_per_step, "eager launches" if args.eager else "graph replays",
                                                      ev_ms, len(steps), n_ops, bound_s * 1e3),
          file=sys.stderr)
    print("bench: first pass incl. H2D/D2H and launch setup %.1f ms; with H2D/D2H median of %d: %.1f ms; "
          "a batch of %d with the host's staging overlapped: %.2f ms/image"
          % (e2e_first * 1e3, len(e2e), e2e_rec["median_ms"], nb, batch_s * 1e3), file=sys.stderr)
    if passes:
        print("bench: per-pass events: median %.3f ms (min %.3f, max %.3f, %d passes)"
              % (passes["median_ms"], passes["min_ms"], passes["max_ms"], passes["n"]), file=sys.stderr)
    print("bench: fused program's roofline bound %.2f ms over %d launches: the pass runs at %.2f of it"
          % (prog_bound_ms, len(launches), prog_bound_ms / ms_per_step), file=sys.stderr)
    fams = collections.defaultdict(lambda: [0.0, 0])
    for k, v in per_kernel.items():
        fams[family(k)][0] += v[0]
        fams[family(k)][1] += v[1]
    tot = sum(v[0] for v in per_kernel.values())
    print("  by family: " + ", ".join("%s %.1f%%" % (k, 100 * v[0] / tot)
                                      for k, v in sorted(fams.items(), key=lambda kv: -kv[1][0])), file=sys.stderr)
    for k, (t, n, f, b, _) in sorted(per_kernel.items(), key=lambda kv: -kv[1][0])[:24]:
        avg = t / n / 1e3
        print("  %-26s %5.1f%%  %4d launches/step  avg %7.1f us  %7.2f TFLOP/s  %7.1f GB/s"
              % (k, 100 * t / tot, n // args.steps, avg * 1e6, f / n / avg / 1e12, b / n / avg / 1e9),
              file=sys.stderr)

    dev_arena = gpu.arena_bytes
    cus, clk = gpu.device_info()
    device = {"name": gpu.device_name, "arch": "gfx950", "cus": cus, "clock_mhz": clk // 1000}
    validation = {"replay_equals_first_pass": same}
    cpu = None
    if not args.no_cpu:
        cpu, ref = cpu_baseline(plan, pad.img, args.cpu_threads, name)
        err = float(np.abs(out_last.astype(np.float64) - ref).max())
        mse = float(((np.clip(out_last, 0, 1) - np.clip(ref, 0, 1)).astype(np.float64) ** 2).mean())
        validation["max_abs_vs_cpu"] = err
        validation["psnr_db_vs_cpu"] = 10 * np.log10(1.0 / mse) if mse > 0 else float("inf")
    gpu.close()
    c5 = None if args.no_c5 else c5_leg(w, R, name)

    line = {
        "metric": METRIC.replace("MAXIM-3S", name),
        "value": 1e3 / ms_per_step,
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: seeded He-normal x0.3 weights, 600x400 smooth pattern + N(0,0.1) image",
        "config": {"workload": "C4: %s, 600x400 RGB reflect-padded to 640x448, one image per step" % name,
                   "variant": args.variant, "ops": n_ops, "launch": "eager" if args.eager else "graph",
                   "arena_mib": round(plan.arena_bytes / 2**20, 1),
                   "device_arena_mib": round(dev_arena / 2**20, 1),
                   "gflop_per_image": round(fl_all / 1e9, 1), "gb_per_image": round(by_all / 1e9, 2),
                   "sum_of_op_bounds_ms": round(bound_s * 1e3, 2)},
        "passes": passes,
        "e2e": e2e_rec,
        "program_roofline": {"bound_ms": prog_bound_ms, "kernel_ms": ev_ms, "launches": len(launches),
                             "frac": prog_bound_ms / ms_per_step,
                             "what": "sum over the fused program's launches of max(FLOPs / 157.3 TFLOP/s, "
                                     "bytes / 8 TB/s), algorithmic accounting; frac = bound / ms_per_step"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "device": device,
        "c5": c5,
        "validation": validation,
    }
    print(json.dumps(line), flush=True)
    bad = not same or ("max_abs_vs_cpu" in validation and (validation["max_abs_vs_cpu"] > 2e-3 or
                                                           validation["psnr_db_vs_cpu"] < 50.0))
    if bad:
        print("bench: the timed passes do not reproduce the reference output: %s" % validation, file=sys.stderr)
        sys.exit(1)


def model_name(variant):
    """S-3 -> MAXIM-3S, M-2 -> MAXIM-2M: the reference's names for the variants."""
    return "MAXIM-%s%s" % (variant[2], variant[0])


def host_threads():
    """The host cores this process may use (OMP_NUM_THREADS when the host
    sets it, as the GPU boxes do, else every core)."""
    try:
        return max(1, int(os.environ["OMP_NUM_THREADS"]))
    except (KeyError, ValueError):
        return os.cpu_count() or 1


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def c5_leg(w, R, name, steps=3):
    """C5: MAXIM-3S on a 4096x4096 image (uniform [0, 1) plus N(0, 0.05),
    clipped), the same weights: ms/image over graph replays, the dominant
    kernel's rate (its tensors are far larger than the Infinity Cache, so its
    HBM figure is cache-free), the whole pass's effective rate, the fused
    program's roofline bound and a per-kernel table."""
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    rng = np.random.default_rng(5)
    img = np.clip(rng.random((3, 4096, 4096)) + rng.normal(0, 0.05, (3, 4096, 4096)), 0, 1).astype(np.float32)
    plan = P.Plan(w, 4096, 4096)
    print("bench: C5 4096x4096, arena %.1f GiB" % (plan.arena_bytes / 2**30), file=sys.stderr, flush=True)
    gpu = H.Gpu(plan)
    try:
        out = gpu.run(img)
        assert np.isfinite(out).all(), "non-finite C5 output"
        gpu.run_graph()
        gpu.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            gpu.run_graph()
        gpu.sync()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        launches = gpu.launches()
        cost = launch_costs(plan, gpu.steps(), launches, R, gpu.launch_spans())
        _, tot = gpu.run_timed()
        lt = gpu.launch_timeline()
        per = collections.defaultdict(lambda: [0.0, 0, 0.0, 0.0, 0.0])
        for k, (st, kn) in enumerate(launches):
            e = per[kn]
            e[0] += float(lt[k])
            e[1] += 1
            e[2] += cost[k][0]
            e[3] += cost[k][1]
            e[4] += launch_bound_ms(cost[k][0], cost[k][1], R)
        kern, (tms, nl, fl, by, bd) = max(per.items(), key=lambda kv: kv[1][0])
        avg_s = tms / nl / 1e3
        fl_all = sum(c[0] for c in cost)
        by_all = sum(c[1] for c in cost)
        dom = rate(fl, by, nl, avg_s, R)
        dom.update({"kernel": kern, "avg_launch_us": avg_s * 1e6, "launches_per_step": nl,
                    "share_of_pass": tms / tot, "frac_of_own_bound": bd / tms})
        # Per kernel: every memory-bound kernel (below the ridge) and the eight
        # GEMM-shaped kernels with the most time, each against its own peak.
        rows = []
        for k, (t, n, f, b, _) in sorted(per.items(), key=lambda kv: -kv[1][0]):
            if n == 0 or t <= 0 or b <= 0:
                continue
            r = rate(f, b, n, t / n / 1e3, R)
            r.update({"kernel": k, "launches": n, "avg_us": 1e3 * t / n, "share": t / tot})
            rows.append(r)
        mem = [r for r in rows if r["bound"] == "hbm"]
        gemm = [r for r in rows if r["bound"] == "mfma"][:8]
        bound_ms = sum(launch_bound_ms(c[0], c[1], R) for c in cost)
        res = {"workload": "C5: %s, 4096x4096 RGB, one image per step" % name, "ms_per_image": ms,
               "images_per_s": 1e3 / ms, "steps": steps, "arena_gib": round(plan.arena_bytes / 2**30, 2),
               "kernel_ms_per_pass": tot, "tflops_effective": fl_all / (ms * 1e-3) / 1e12,
               "tb_per_s_effective": by_all / (ms * 1e-3) / 1e12,
               "algorithmic_per_pass": {"gflop": fl_all / 1e9, "gb": by_all / 1e9}, "dominant": dom,
               "program_roofline": {"bound_ms": bound_ms, "frac": bound_ms / ms},
               "kernels": {"memory_bound": [compact(r) for r in mem], "gemm_top8": [compact(r) for r in gemm]}}
        print("bench: C5 per kernel (cache-free: every level-0 tensor is 2 GB):", file=sys.stderr)
        for r in mem + gemm:
            print("  %-30s %4d launches  avg %8.1f us  %8.1f %-7s  %.2f of peak  %4.1f%% of the pass"
                  % (r["kernel"], r["launches"], r["avg_us"], r["achieved"], r["unit"], r["frac"],
                     100 * r["share"]), file=sys.stderr)
        print("bench: C5 %.1f ms/image; dominant %s %.1f us x %d (%.1f%% of %s peak)"
              % (ms, kern, avg_s * 1e6, nl, 100 * dom["frac"], dom["unit"]), file=sys.stderr, flush=True)
        return res
    finally:
        gpu.close()


def rate(flops, nbytes, n, avg_s, R):
    """A kernel's achieved rate over n launches of avg_s seconds against the
    peak its arithmetic intensity puts it under (fp32 MFMA above the ridge,
    HBM below)."""
    if nbytes and flops / nbytes >= R.RIDGE:
        r = {"bound": "mfma", "achieved": flops / n / avg_s / 1e12, "peak": 157.3, "unit": "TFLOP/s"}
    else:
        r = {"bound": "hbm", "achieved": nbytes / n / avg_s / 1e9, "peak": 8000.0, "unit": "GB/s"}
    r["frac"] = r["achieved"] / r["peak"]
    return r


def compact(r):
    return {"kernel": r["kernel"], "launches": r["launches"], "avg_us": round(r["avg_us"], 2),
            "bound": r["bound"], "achieved": round(r["achieved"], 2), "unit": r["unit"],
            "frac": round(r["frac"], 3), "share": round(r["share"], 4)}


TRAFFIC = os.path.join(ROOT, "profiles", "hbm_traffic_c4.md")


def traffic_per_launch(kernel):
    """HBM-side bytes per launch of `kernel` at C4, from the committed
    rocprofv3 summary (FETCH_SIZE and WRITE_SIZE passes, each scaled by what
    the counter reads for a copy of known size); None if the kernel is not in
    it."""
    try:
        rows = open(TRAFFIC).read().splitlines()
    except OSError:
        return None
    for r in rows:
        cells = [c.strip() for c in r.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[0] == kernel:
            return float(cells[4]) * 1e6
    return None


def launch_costs(plan, steps, launches, R, spans=None):
    """(flops, bytes) of every launch: FLOPs = 2 x MACs; bytes = what the
    kernel must move (inputs once, output once, weights once). A step of one
    launch is charged its ops' costs less the intermediates it no longer
    writes and reads back; a launch that names its own ops (`spans`: in a
    step pairing two branches' launches, each launch computes one former
    step, or two side by side) is charged as those steps were; the other
    steps of several launches are split by kernel:
    a folded LayerNorm's statistics pass (reads x, writes mean and 1/std) and
    the GEMM that re-reads x with them, the two resize passes through `tmp`,
    the channel mean's partial and final sums, and the partial sums before
    the CALayer block that finishes the means. A GEMM step that ends in the
    LayerNorm of an output band (the _lo kernels) is the GEMM step's cost plus
    the LayerNorm's output, less the band's raw store when nothing else
    reads it."""
    from maxim_amd import plan as P

    def read_later(buf, after):
        """Whether an op after `after` reads buf's bytes before they are rewritten."""
        lo, hi = int(plan.offs[buf]), int(plan.offs[buf]) + plan.buf_len(buf)
        for k in range(after + 1, len(plan.ops)):
            o = plan.ops[k]
            for s in plan.operands(o)[1:]:
                if s >= 0 and int(plan.offs[s]) < hi and lo < int(plan.offs[s]) + plan.buf_len(s):
                    return True
            d = o.dst
            if int(plan.offs[d]) <= lo and hi <= int(plan.offs[d]) + plan.buf_len(d):
                return False
        return False

    def step_cost(a, b):
        ln = plan.ops[b - 1]
        if b - a > 1 and ln.kind == P.CHAN_LN and plan.ops[b - 2].kind != P.CHAN_LN:
            f, by = step_cost(a, b - 1)
            band = 4 * ln.c * ln.hw
            return f, by + band - (0 if read_later(ln.src, b - 1) else band)
        f = sum(R.op_cost(plan.ops[k])[0] for k in range(a, b))
        by = sum(R.op_cost(plan.ops[k])[1] for k in range(a, b))
        by -= sum(8 * plan.buf_len(plan.ops[k].dst) for k in range(a, b - 1))
        return f, by

    per_step = collections.defaultdict(list)
    for i, (st, kn) in enumerate(launches):
        per_step[st].append(i)
    out = [None] * len(launches)
    for st, idx in per_step.items():
        a, b, _ = steps[st]
        o = plan.ops[a]
        names = [launches[i][1] for i in idx]
        if spans is not None and any(spans[i][1] is not None or spans[i][0] != (a, b) for i in idx):
            for i in idx:
                (a0, b0), second = spans[i]
                f, by = step_cost(a0, b0)
                if second is not None:
                    f2, by2 = step_cost(*second)
                    f, by = f + f2, by + by2
                out[i] = (f, by)
            continue
        if len(idx) == 1:
            out[idx[0]] = step_cost(a, b)
            continue
        if o.kind == P.RESIZE and b - a == 2 and plan.ops[a + 1].kind == P.CONV1X1 and len(idx) == 2:
            # a commuted UpSampleRatio: the conv at the resize's input
            # resolution, then the resize of the conv's c_out channels
            c = plan.ops[a + 1]
            pl, opl = o.h * o.wd, o.oh * o.ow
            bias = c.c_out if c.bias >= 0 else 0
            for i, kn in zip(idx, names):
                if kn.startswith("mx_resize"):
                    out[i] = (0, 4 * c.c_out * (pl + opl))
                else:
                    out[i] = (2 * c.c_in * c.c_out * pl, 4 * (c.c_in * pl + c.c_out * pl + c.c_in * c.c_out + bias))
            continue
        if o.kind == P.CONV4X4S2 and len(idx) == 2:
            # a split-reduction 4x4: the slices carry the op's work, their
            # sum (mx_conv_split_sum) moves only partials
            for i, kn in zip(idx, names):
                out[i] = step_cost(a, b) if kn.startswith("mx_conv4x4") else (0, 0)
            continue
        for i, kn in zip(idx, names):
            if kn.startswith("mx_chan_ln_stats"):
                out[i] = (0, 4 * (o.c * o.hw + 2 * o.hw))
            elif kn.startswith("mx_pw_") and "_ln" in kn:
                f, by = step_cost(a, b)
                out[i] = (f, by + 8 * o.hw)  # + the statistics it reads
            elif kn.startswith("mx_chan_ln"):  # a LayerNorm that could not be folded
                last = plan.ops[b - 1]
                out[i] = R.op_cost(last if b - 1 > a and last.kind == P.CHAN_LN else o)
            elif kn == "mx_resize_h":
                out[i] = (0, 4 * (o.c * o.h * o.wd + o.c * o.h * o.ow))
            elif kn == "mx_resize_v":
                out[i] = (0, 4 * (o.c * o.h * o.ow + o.c * o.oh * o.ow))
            elif kn.startswith("mx_chan_mean_part"):
                out[i] = (0, 4 * o.c * o.hw)
            elif kn == "mx_chan_mean_final":
                out[i] = (0, 4 * o.c)
            elif kn == "mx_ca_mean_mlp":  # the means finished, then the CALayer MLP
                f, by = step_cost(a + 1, b)
                out[i] = (f, by + 4 * o.c)
            else:  # the GEMM after an unfolded LayerNorm
                out[i] = step_cost(a + 1, b)
    return out


def cpu_baseline(plan, img, threads, name="MAXIM-3S"):
    """The CPU path (oracle/: a C restatement of src/exec_cpu.rs, OpenMP over
    channels, rows and pixels) on this host: the median of three full C4
    passes on `threads` cores, and one single-thread C1 pass (MAXIM-2S,
    256x256) for scaling. Returns the record and the C4 output."""
    from oracle import oracle as O
    from maxim_amd import plan as P

    def one(pl, im, th):
        arena = np.zeros(pl.arena_len, np.float32)
        o = int(pl.offs[pl.input])
        arena[o:o + im.size] = im.ravel()
        t0 = time.perf_counter()
        O.run(pl, arena, th)
        dt = time.perf_counter() - t0
        q = int(pl.offs[pl.output])
        c, h, w = pl.bufs[pl.output]
        return dt, arena[q:q + c * h * w].reshape(c, h, w).copy()

    times, ref = [], None
    for _ in range(3):
        dt, ref = one(plan, img, threads)
        times.append(dt)
    used = O.threads_used()
    med = float(np.median(times))
    w2 = P.Weights.synthetic("S-2", seed=SEED, gain=GAIN, bias_std=0.02, ln_std=0.1)
    c1 = P.Plan(w2, 256, 256)
    dt1, _ = one(c1, np.random.default_rng(2).random((3, 256, 256), dtype=np.float32), 1)
    # C2: the first split-head gMLP layer of the MAXIM-2S 256x256 plan (its 25
    # ops, LayerNorm_in through the residual add), x ~ N(0, 1), one thread
    c2 = P.Plan(w2, 256, 256, named=True, deep=True)
    first, last, x = gmlp_layer_range(c2)
    arena = np.zeros(c2.arena_len, np.float32)
    arena[int(c2.offs[x]):int(c2.offs[x]) + c2.buf_len(x)] = \
        np.random.default_rng(8).standard_normal(c2.buf_len(x)).astype(np.float32)
    t0 = time.perf_counter()
    O.run_range(c2, arena, first, last, 1)
    dt2 = time.perf_counter() - t0
    print("bench: CPU C4 %s s on %d threads, C1 %.1f s and C2 %.2f s on 1 thread (%s)"
          % (", ".join("%.2f" % t for t in times), used, dt1, dt2, cpu_model()), file=sys.stderr, flush=True)
    rec = {"value": 1.0 / med, "unit": "images/s", "cores": used, "kind": "port",
           "sample": "median of 3 full %s 640x448 passes (%d ops) of the C restatement of src/exec_cpu.rs: %s s"
                     % (name, len(plan.ops), ", ".join("%.2f" % t for t in times)),
           "cpu_model": cpu_model(), "host_cores_visible": os.cpu_count(),
           "c1_single_thread": {"seconds": dt1, "images_per_s": 1.0 / dt1,
                                "workload": "C1: MAXIM-2S 256x256, one pass, 1 thread"},
           "c2_single_thread": {"seconds": dt2, "ops": last - first,
                                "workload": "C2: one split-head gMLP layer (c=32, 256x256, block 16 + grid 16), "
                                            "1 thread"}}
    return rec, ref


def gmlp_layer_range(plan):
    """(first, last, x): the ops of the first split-head gMLP layer of a
    `named` MAXIM plan - after the first encoder block's Conv_0 (buffer x)
    through the layer's residual add."""
    d = dict(plan.dumps)
    x = d["stage_0_encoder_block_0_mid_conv"]
    y = d["stage_0_encoder_block_0_mid_g0_gmlp"]
    first = next(i for i, op in enumerate(plan.ops) if op.dst == x) + 1
    last = next(i for i, op in enumerate(plan.ops) if op.dst == y) + 1
    return first, last, x


def launch_bound_ms(flops, nbytes, R):
    """A launch's roofline time: the larger of its FLOPs at the fp32 MFMA peak
    and its bytes at the HBM peak (ms)."""
    return 1e3 * max(flops / R.PEAK_FP32_MFMA, nbytes / R.PEAK_HBM)


if __name__ == "__main__":
    main()
