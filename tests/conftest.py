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


# Per-op bars of the lockstep walks (the reference's --verify-gpu uses
# max|d| <= 1e-3 * max|cpu| for every op, src/main.rs:709-712):
#   exact     ops whose arithmetic the executor reproduces term for term
#   ulps      gelu (fitted exp2 polynomial vs libm erff), sigmoid (hardware exp2
#             and reciprocal vs libm expf):
#             |d| <= 4e-7 * (1 + |x|)
#   rounding  chan_mean and every matrix-core GEMM: max|d| <= 1e-4 * max|cpu|
EXACT = {"copy", "add", "mul", "gate_apply", "lrelu", "chan_scale", "chan_ln", "block_perm",
         "down_s", "resize"}
ULPS = {"gelu", "sigmoid"}


def op_sources(plan, op):
    """The arena buffers an op reads (a resize's second operand is its scratch)."""
    from maxim_amd import plan as P
    return [op.src] if op.kind == P.RESIZE else plan.operands(op)[1:]


def _max_abs_diff(got, want, x=None, chunk=1 << 25):
    """max |got - want| (divided by 1 + |x| where x is given) in float64, in
    chunks, so that billion-element buffers need no billion-element
    temporaries."""
    m = 0.0
    for a in range(0, want.size, chunk):
        d = np.abs(got[a:a + chunk].astype(np.float64) - want[a:a + chunk])
        if x is not None:
            d /= 1.0 + np.abs(x[a:a + chunk].astype(np.float64))
        if d.size:
            m = max(m, float(d.max()))
    return m


def judge_op(plan, arena, op, got):
    """(ok, kind key, error) of the device result `got` for `op` against the
    oracle's result already in `arena`."""
    from maxim_amd import plan as P
    name = P.OP_NAMES[op.kind]
    want = buf(plan, arena, op.dst)
    if op.kind in (P.COPY, P.GELU, P.LRELU, P.SIGMOID):
        want = want[:op.n]
    got = got[:want.size]
    exact = name in EXACT or (op.kind == P.CONV1X1 and op.h * op.wd == 1)
    if exact:
        ok = np.array_equal(got.view(np.uint32), want.view(np.uint32))
        if not ok:
            ok = np.array_equal(got, want) and not np.isnan(want).any()
        rel = 0.0 if ok else _max_abs_diff(got, want)
    elif name in ULPS:
        rel = _max_abs_diff(got, want, buf(plan, arena, op.src)[:op.n])
        ok = rel <= 4e-7
    else:
        scale = float(np.abs(want).max()) if want.size else 0.0
        rel = _max_abs_diff(got, want)
        rel = rel / scale if scale > 0 else rel
        ok = rel <= 1e-4
    key = "gemv" if exact and op.kind == P.CONV1X1 else name
    return ok, key, rel


def rewrite_safetensors(path, new_value):
    """Overwrite tensors of a safetensors file in place: new_value(name,
    array) returns the replacement (same shape, float32) or None to keep the
    tensor. The header is unchanged, so the file stays a valid checkpoint."""
    import json
    import struct
    with open(path, "r+b") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
        base = 8 + n
        for name, meta in header.items():
            if name == "__metadata__":
                continue
            assert meta["dtype"] == "F32", meta
            b, e = meta["data_offsets"]
            f.seek(base + b)
            old = np.frombuffer(f.read(e - b), np.float32).reshape(meta["shape"])
            new = new_value(name, old)
            if new is None:
                continue
            new = np.ascontiguousarray(new, np.float32)
            assert new.shape == old.shape, (name, new.shape, old.shape)
            f.seek(base + b)
            f.write(new.tobytes())
