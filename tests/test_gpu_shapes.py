"""Whole passes at plan shapes unlike the benchmark's: tall and wide images,
and levels whose grid and block cells take other widths (so other kernel
forms, elided or launched permutations and other pairing windows), each
against the CPU path at the whole-image bar (max-abs 2e-3, PSNR >= 50 dB),
with the two properties the timed path rests on checked at every shape:
graph replays give the eager pass's bits, and the paired launches give the
unpaired program's bits (MAXIM_NO_PAIR=1)."""

import numpy as np
import pytest

from conftest import buf, psnr, run_oracle, smooth_image, weights

pytestmark = pytest.mark.gpu

SHAPES = [("S-3", 64, 320), ("S-3", 192, 64), ("S-3", 320, 192), ("S-2", 128, 448), ("M-1", 192, 128)]


@pytest.mark.parametrize("variant,h,w", SHAPES)
def test_whole_pass_at_unusual_shapes(gpu_ok, variant, h, w, monkeypatch):
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    plan = P.Plan(weights(variant), h, w)
    img = smooth_image(h, w, seed=h + w)
    print("%s %dx%d: %d ops" % (variant, h, w, len(plan.ops)), flush=True)
    gpu = H.Gpu(plan)
    try:
        out = gpu.run(img).copy()
        paired = sum(1 for _, k in gpu.launches() if k.endswith("_x2"))
        gpu.set_graph(True)
        replay = gpu.run(img).copy()
    finally:
        gpu.close()
    ref = buf(plan, run_oracle(plan, img), plan.output).reshape(out.shape)
    err = float(np.abs(out.astype(np.float64) - ref).max())
    print("%s %dx%d: %d paired launches, max-abs %.3g, PSNR %.1f dB"
          % (variant, h, w, paired, err, psnr(out, ref)), flush=True)
    assert np.isfinite(out).all()
    assert err <= 2e-3 and psnr(out, ref) >= 50.0
    assert np.array_equal(replay.view(np.uint32), out.view(np.uint32))
    monkeypatch.setenv("MAXIM_NO_PAIR", "1")
    gpu = H.Gpu(plan)
    try:
        assert not any(k.endswith("_x2") for _, k in gpu.launches())
        unpaired = gpu.run(img)
    finally:
        gpu.close()
    assert np.array_equal(unpaired.view(np.uint32), out.view(np.uint32))
