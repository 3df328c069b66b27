"""The dump comparison of the package's dev tools (tools/compare.py): RMS
above the tolerance is a failure, shapes must agree after dropping a
leading singleton, and tensors are ordered by stage and level."""

import numpy as np
import pytest


def test_compare_dumps(tmp_path):
    from maxim_amd import devtools as D
    a, b = tmp_path / "ref", tmp_path / "mine"
    a.mkdir()
    b.mkdir()
    rng = np.random.default_rng(0)
    names = ["stage_10_x", "stage_2_x", "stage_1_enc_0"]
    for n in names:
        x = rng.random((3, 8, 8)).astype(np.float32)
        np.save(a / (n + ".npy"), x[None])          # the reference dumps NCHW
        np.save(b / (n + ".npy"), x + np.float32(1e-6))
    rows, failures = D.compare_dumps(str(a), str(b), out=lambda s: None)
    assert failures == 0 and [r[0] for r in rows] == ["stage_1_enc_0", "stage_2_x", "stage_10_x"]
    assert all(abs(r[3] - 1e-6) < 1e-7 for r in rows)
    np.save(b / "stage_2_x.npy", np.load(a / "stage_2_x.npy")[0] + np.float32(1e-3))
    np.save(b / "stage_10_x.npy", np.zeros((3, 4, 4), np.float32))
    seen = []
    rows, failures = D.compare_dumps(str(a), str(b), out=seen.append)
    assert failures == 2 and any("SHAPE" in s for s in seen) and any("FAIL" in s for s in seen)
    assert D.main(["compare", str(a), str(b)]) == 1
    with pytest.raises(ValueError):
        D.compare_dumps(str(a), str(tmp_path))
