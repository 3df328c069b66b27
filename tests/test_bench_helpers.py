"""The benchmark's host-side helpers (no GPU): the C2 layer range the CPU
baseline times, and the per-launch roofline bound the program's bound sums."""

import pytest

from conftest import weights


def test_c2_range_is_the_split_head_layer():
    import bench
    from maxim_amd import plan as P
    plan = P.Plan(weights("S-2"), 256, 256, named=True, deep=True)
    first, last, x = bench.gmlp_layer_range(plan)
    assert last - first == 25 and plan.bufs[x] == (32, 256, 256)
    kinds = [plan.ops[i].kind for i in range(first, last)]
    assert kinds[0] == P.CHAN_LN and kinds[-1] == P.ADD
    assert kinds.count(P.GATE_MM) == 2


def test_launch_bound_is_the_larger_of_compute_and_memory():
    import bench
    from maxim_amd import roofline as R
    # 157.3 GFLOP alone: 1 ms at the MFMA peak; 8 GB alone: 1 ms at the HBM peak
    assert bench.launch_bound_ms(157.3e9, 0, R) == pytest.approx(1.0)
    assert bench.launch_bound_ms(0, 8e9, R) == pytest.approx(1.0)
    assert bench.launch_bound_ms(157.3e9, 16e9, R) == pytest.approx(2.0)
    r = bench.rate(2 * 157.3e9, 1e9, 2, 1e-3, R)  # above the ridge: the MFMA axis
    assert r["bound"] == "mfma" and r["frac"] == pytest.approx(1.0)
    r = bench.rate(1e9, 8e9, 1, 2e-3, R)  # below it: HBM
    assert r["bound"] == "hbm" and r["frac"] == pytest.approx(0.5)
