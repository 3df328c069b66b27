"""Gpu::new's refusal (src/exec_gpu.rs:86-146): a plan whose arena and
weights exceed the device's free memory is refused up front, with the
numbers, and the refusal costs nothing - everything the executor created
before it (stream, arena, weights, scratch) is released, so a caller can
retry at a smaller size with the device as it was."""

import numpy as np
import pytest

from conftest import weights

pytestmark = pytest.mark.gpu


def test_over_limit_plan_is_refused_with_the_numbers_and_frees_everything():
    from maxim_amd import hip as H
    from maxim_amd import plan as P
    w = weights("S-3")
    # load the code object (kept per device) before taking the baseline
    small = H.Gpu(P.Plan(w, 64, 64))
    small.close()
    free0, total = H.device_memory()
    huge = P.Plan(w, 16384, 16384)  # an arena of ~460 GiB
    assert huge.arena_bytes > total, (huge.arena_bytes, total)
    print("refusal: S-3 16384x16384, arena %.1f GiB, device %.1f GiB" % (huge.arena_bytes / 2**30, total / 2**30),
          flush=True)
    for _ in range(3):
        with pytest.raises(P.MaximError) as e:
            H.Gpu(huge)
        msg = str(e.value)
        assert "not enough device memory" in msg and "MiB" in msg and "is free" in msg, msg
    free1, _ = H.device_memory()
    assert abs(int(free1) - int(free0)) <= 8 << 20, (free0, free1)
    # and the device still runs a pass
    g = H.Gpu(P.Plan(w, 64, 64))
    try:
        out = g.run(np.random.default_rng(3).random((3, 64, 64), dtype=np.float32))
        assert np.isfinite(out).all()
    finally:
        g.close()
