"""--dump on the device (src/image.rs:250-269) and its comparison with the
CPU path's activations (tools/compare.py): every named activation of the
`named` plan, RMS within 1e-4."""

import numpy as np
import pytest

from conftest import buf, run_oracle, smooth_image, weights

pytestmark = pytest.mark.gpu


def test_dump_and_compare_with_the_cpu_path(gpu_ok, tmp_path):
    from maxim_amd import devtools as D
    from maxim_amd import hip as H
    from maxim_amd import plan as P
    plan = P.Plan(weights("S-2"), 64, 64, named=True)
    img = smooth_image(64, 64, seed=2)
    gpu = H.Gpu(plan)
    gpu.run(img)
    paths = D.dump_named(gpu, plan, str(tmp_path / "gpu"))
    gpu.close()
    assert len(paths) == len(plan.dumps) >= 40
    arena = run_oracle(plan, img)
    cpu = tmp_path / "cpu"
    cpu.mkdir()
    for name, b in plan.dumps:
        np.save(cpu / (D.dump_name(name) + ".npy"), buf(plan, arena, b).reshape(plan.bufs[b]))
    rows, failures = D.compare_dumps(str(cpu), str(tmp_path / "gpu"), out=print)
    assert failures == 0 and len(rows) == len(paths)
    worst = max(r[3] for r in rows)
    print("worst RMS %.3g over %d tensors" % (worst, len(rows)))
