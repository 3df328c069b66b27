"""python -m maxim_amd: the enhancement run with the reference's development
flags (src/main.rs:20-58 and 173-458 with `--features dev`), on the MI355X.

    python -m maxim_amd -m MODEL.safetensors [-i IN.png|-] [-o OUT.png|-]
                        [--dump DIR] [--profile] [--factor N] [-q]

  --dump DIR   every named activation of the pass as DIR/<name>.npy
               (src/image.rs:250-269; the plan is built `named`, which keeps
               those buffers), for `python -m maxim_amd.devtools compare`
  --profile    the per-op census (op families, shapes, slowest ops) and the
               fused program's kernels (src/main.rs:526-656); also --timeline
  --factor N   pad to a multiple of N instead of 64 (src/image.rs:171-207)

The pass is the one `maxim_hip` and mxh_enhance run (checkpoint, even-ize and
reflect-pad, the plan, the device pass, the crop). --verify-gpu steps the
CPU path beside the device; this package has no CPU path of its own, so the
walk is `devtools.verify_walk(plan, image, cpu_step)` with the caller's CPU
step, and the flag is refused here by name. So are --device cpu and --cpu.
"""

import argparse
import sys
import time

from . import devtools as D
from . import hip as H
from . import plan as P


def parse(argv):
    ap = argparse.ArgumentParser(prog="python -m maxim_amd", add_help=False)
    ap.add_argument("-m", "--model")
    ap.add_argument("-i", "--input", default="-")
    ap.add_argument("-o", "--output", default="-")
    ap.add_argument("--device", default="gpu")
    ap.add_argument("--gpu", action="store_true")
    ap.add_argument("--cpu", action="store_true")
    ap.add_argument("-q", "--quiet", action="store_true")
    ap.add_argument("--dump")
    ap.add_argument("--profile", "--timeline", action="store_true", dest="profile")
    ap.add_argument("--verify-gpu", action="store_true", dest="verify")
    ap.add_argument("--factor", type=int, default=64)
    ap.add_argument("-h", "--help", action="store_true")
    return ap, ap.parse_args(argv)


def main(argv=None):
    ap, a = parse(sys.argv[1:] if argv is None else argv)
    if a.help:
        print(__doc__, file=sys.stderr)
        return 2
    if a.cpu or a.device not in ("gpu", "hip"):
        print("maxim: this package runs on the MI355X only (no CPU backend)", file=sys.stderr)
        return 2
    if a.verify:
        print("maxim: --verify-gpu needs a CPU path; call maxim_amd.devtools.verify_walk with one",
              file=sys.stderr)
        return 2
    if not a.model:
        print("maxim: --model is required", file=sys.stderr)
        return 2
    if a.factor <= 0:
        print("maxim: --factor must be positive", file=sys.stderr)
        return 2
    log = (lambda *x: None) if a.quiet else (lambda *x: print("maxim:", *x, file=sys.stderr, flush=True))
    try:
        img = P.read_png(data=sys.stdin.buffer.read()) if a.input == "-" else P.read_png(a.input)
        weights = P.Weights.open(a.model)
        padded = P.preprocess(img, a.factor)
        _, ph, pw = padded.img.shape
        plan = P.Plan(weights, ph, pw, named=bool(a.dump))
        log("%dx%d padded to %dx%d, %d ops, arena %.1f MiB"
            % (img.shape[2], img.shape[1], pw, ph, len(plan.ops), plan.arena_bytes / 2**20))
        gpu = H.Gpu(plan)
        try:
            t0 = time.perf_counter()
            out = gpu.run(padded.img)
            log("pass in %.2fs on %s" % (time.perf_counter() - t0, gpu.device_name))
            if a.dump:
                paths = D.dump_named(gpu, plan, a.dump)
                log("wrote %d activations to %s" % (len(paths), a.dump))
        finally:
            gpu.close()
        if a.profile:
            D.timeline_report(plan, padded.img, out=lambda s: print(s, file=sys.stderr))
        res = P.crop_out(out, padded)
        if a.output == "-":
            sys.stdout.buffer.write(P.encode_png(res))
            sys.stdout.buffer.flush()
        else:
            P.write_png(a.output, res)
            log("wrote %s" % a.output)
    except (P.MaximError, OSError) as e:
        print("maxim: %s" % e, file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
