import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "maxim-rs_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP executor)")
    config.addinivalue_line("markers", "slow: long-running CPU oracle case")
    lib = os.path.join(ROOT, "maxim-rs_amd", "lib", "libmaxim_hip.so")
    orc = os.path.join(ROOT, "oracle", "liboracle.so")
    if not (os.path.exists(lib) and os.path.exists(orc)):
        import __graft_entry__
        __graft_entry__.build()


_WEIGHTS = {}


def weights(variant="S-2", seed=1, gain=0.3, bias_std=0.02, ln_std=0.1):
    """Seeded random-init weights, cached per process (they take ~1 s)."""
    from maxim_amd import plan as P
    key = (variant, seed, gain, bias_std, ln_std)
    if key not in _WEIGHTS:
        _WEIGHTS[key] = P.Weights.synthetic(variant, seed=seed, gain=gain, bias_std=bias_std, ln_std=ln_std)
    return _WEIGHTS[key]


def smooth_image(h, w, seed=0, noise=0.1):
    """A low-frequency pattern plus Gaussian noise, clipped to [0, 1]."""
    rng = np.random.default_rng(seed)
    y, x = np.mgrid[0:h, 0:w].astype(np.float64)
    img = np.empty((3, h, w))
    for c in range(3):
        f = rng.uniform(0.5, 3.0, size=(3, 2))
        ph = rng.uniform(0, 2 * np.pi, size=3)
        v = 0.5 + sum(0.1 * np.sin(2 * np.pi * (f[k, 0] * y / h + f[k, 1] * x / w) + ph[k]) for k in range(3))
        img[c] = v + rng.normal(0, noise, size=(h, w))
    return np.clip(img, 0, 1).astype(np.float32)


def run_oracle(plan, img, threads=0):
    from oracle import oracle as O
    arena = np.zeros(plan.arena_len, np.float32)
    o = int(plan.offs[plan.input])
    arena[o:o + img.size] = img.ravel()
    O.run(plan, arena, threads)
    return arena


def buf(plan, arena, b):
    o = int(plan.offs[b])
    return arena[o:o + plan.buf_len(b)]


def psnr(a, b):
    mse = float(((np.clip(a, 0, 1).astype(np.float64) - np.clip(b, 0, 1)) ** 2).mean())
    return float("inf") if mse == 0 else 10 * np.log10(1.0 / mse)


@pytest.fixture(scope="session")
def gpu_ok():
    from maxim_amd import hip as H
    if not H.driver_ready():
        pytest.fail("no HIP device: the gpu tests need an MI355X")
    return True
