"""The enhancement run end to end from files, on the device: a checkpoint
written in the reference's safetensors layout and read back (the variant
comes from the file, src/weights.rs:37-41, src/config.rs:71-100), a PNG
input, the reference pipeline's padding, the HIP pass and the crop
(src/main.rs:173-458) - through mxh_enhance and through the maxim_hip
command - against the CPU path on the same file and pixels, at the
north-star bar (max-abs 2e-3, PSNR >= 50 dB; the 8-bit outputs within one
level)."""

import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, psnr, run_oracle, smooth_image, weights

pytestmark = pytest.mark.gpu


def test_c4_from_checkpoint_and_png(gpu_ok, tmp_path):
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    ckpt = str(tmp_path / "maxim_s3.safetensors")
    weights("S-3").save(ckpt)
    src = str(tmp_path / "in.png")
    P.write_png(src, smooth_image(400, 600, seed=4))
    img = P.read_png(src)
    assert img.shape == (3, 400, 600)
    print("checkpoint: S-3 from file, 600x400 PNG", flush=True)
    got = H.enhance(ckpt, img)

    # the CPU path on the same file and pixels
    w = P.Weights.open(ckpt)
    assert w.config.num_stages == 3 and w.params == weights("S-3").params
    pad = P.preprocess(img, 64)
    plan = P.Plan(w, *pad.img.shape[1:])
    arena = run_oracle(plan, pad.img)
    o = int(plan.offs[plan.output])
    pred = arena[o:o + pad.img.size].reshape(pad.img.shape)
    ref = P.crop_out(pred, pad)
    err = float(np.abs(got.astype(np.float64) - ref).max())
    print("mxh_enhance vs CPU path: max-abs %.3g, PSNR %.1f dB" % (err, psnr(got, ref)), flush=True)
    assert got.shape == (3, 400, 600) and err <= 2e-3 and psnr(got, ref) >= 50.0

    # the command: PNG in, PNG out
    out = str(tmp_path / "out.png")
    exe = os.path.join(ROOT, "maxim-rs_amd", "lib", "maxim_hip")
    r = subprocess.run([exe, "-m", ckpt, "-i", src, "-o", out], capture_output=True, text=True, timeout=300)
    print(r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    cli = P.read_png(out)
    want = str(tmp_path / "want.png")
    P.write_png(want, ref)
    levels = np.abs(np.rint(cli * 255) - np.rint(P.read_png(want) * 255))
    print("maxim_hip vs CPU path: %d of %d samples one level apart" % (int((levels > 0).sum()), levels.size))
    assert levels.max() <= 1.0


def test_enhance_refuses_a_bad_checkpoint(gpu_ok, tmp_path):
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    bad = str(tmp_path / "bad.safetensors")
    open(bad, "wb").write(b"\x08\x00\x00\x00\x00\x00\x00\x00{}      ")
    with pytest.raises(P.MaximError):
        H.enhance(bad, np.zeros((3, 64, 64), np.float32))


def test_cli_stdin_stdout_interlaced(gpu_ok, tmp_path):
    """`maxim_hip -m CKPT` with the image on stdin and the result on stdout
    (`-i -` / `-o -`, and the same with both options absent, as
    src/main.rs:205-214,439-448), the input an Adam7-interlaced RGBA PNG of
    an odd size, against the CPU path at the 8-bit bar."""
    from maxim_amd import plan as P
    from test_png import write_interlaced_png
    ckpt = str(tmp_path / "maxim_s2.safetensors")
    weights("S-2").save(ckpt)
    img = smooth_image(70, 90, seed=9)
    px = np.concatenate([np.rint(img * 255).astype(np.uint8).transpose(1, 2, 0),
                         np.full((70, 90, 1), 200, np.uint8)], axis=2)
    src = str(tmp_path / "in_a7.png")
    write_interlaced_png(src, px, 6, 6)
    got = P.read_png(src)
    assert np.array_equal(got, np.rint(img * 255).astype(np.float32) / np.float32(255.0))
    pad = P.preprocess(got, 64)
    plan = P.Plan(P.Weights.open(ckpt), *pad.img.shape[1:])
    arena = run_oracle(plan, pad.img)
    o = int(plan.offs[plan.output])
    ref = P.crop_out(arena[o:o + pad.img.size].reshape(pad.img.shape), pad)
    want = np.rint(np.clip(ref, 0, 1) * 255)
    exe = os.path.join(ROOT, "maxim-rs_amd", "lib", "maxim_hip")
    data = open(src, "rb").read()
    for args in (["-i", "-", "-o", "-"], []):
        print("maxim_hip %s (stdin -> stdout)" % " ".join(args), flush=True)
        r = subprocess.run([exe, "-m", ckpt, "-q"] + args, input=data, capture_output=True, timeout=300)
        assert r.returncode == 0, r.stderr.decode()
        out = P.read_png(data=r.stdout)
        assert out.shape == (3, 70, 90)
        assert np.abs(np.rint(out * 255) - want).max() <= 1.0


def test_dev_entry_point_dump_profile(gpu_ok, tmp_path):
    """`python -m maxim_amd` (the reference's dev build: src/main.rs with
    --dump and --profile) gives the same PNG as `maxim_hip` on the same
    checkpoint and image (byte for byte; with --dump the plan is built
    `named`, whose kept buffers can change which ops fuse, so there within
    one 8-bit level), writes every named activation as .npy and prints the
    census; stdin/stdout work as they do for the command."""
    import sys
    from maxim_amd import plan as P
    ckpt = str(tmp_path / "maxim_s2.safetensors")
    weights("S-2").save(ckpt)
    src = str(tmp_path / "in.png")
    P.write_png(src, smooth_image(100, 140, seed=3))
    exe = os.path.join(ROOT, "maxim-rs_amd", "lib", "maxim_hip")
    ref_png = str(tmp_path / "ref.png")
    r = subprocess.run([exe, "-m", ckpt, "-i", src, "-o", ref_png, "-q"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, PYTHONPATH=os.path.join(ROOT, "maxim-rs_amd"))
    dump = str(tmp_path / "dump")
    out_png = str(tmp_path / "out.png")
    print("python -m maxim_amd --dump --profile", flush=True)
    r = subprocess.run([sys.executable, "-m", "maxim_amd", "-m", ckpt, "-i", src, "-o", out_png,
                        "--dump", dump, "--profile"], capture_output=True, text=True, timeout=600, env=env)
    print(r.stderr[-3000:], flush=True)
    assert r.returncode == 0, r.stderr
    levels = np.abs(np.rint(P.read_png(out_png) * 255) - np.rint(P.read_png(ref_png) * 255))
    assert levels.max() <= 1.0
    files = sorted(os.listdir(dump))
    assert len(files) >= 40 and all(f.endswith(".npy") for f in files), files[:5]
    assert "fused program:" in r.stderr and "slowest ops:" in r.stderr
    r = subprocess.run([sys.executable, "-m", "maxim_amd", "-m", ckpt, "-q"], input=open(src, "rb").read(),
                       capture_output=True, timeout=600, env=env)
    assert r.returncode == 0, r.stderr.decode()
    assert r.stdout == open(ref_png, "rb").read()
