"""Pins the CPU oracle (oracle/exec_cpu.c) - the checker every GPU parity test
trusts - against what fixes each arm independently of its own code:
library routines (torch CPU conv2d / conv_transpose2d / interpolate in
float64), float64 closed forms, numpy index maps taken from the reference's
transcription (tools/reference.py:174-217), and special cases. Each check is
chosen so that a plausible slip (a dropped bias, a transposed weight, an
unbiased variance, a missing antialias widening, an off-by-half sample
position, swapped gate operands) fails it.
"""

import math

import numpy as np
import pytest

from conftest import buf, run_oracle, weights


def O():
    from oracle import oracle
    return oracle


def rng(seed):
    return np.random.default_rng(seed)


def rel_err(got, want):
    want = np.asarray(want, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


# ------------------------------------------------------------ elementwise

def test_binary_ops_are_exact_closed_forms():
    a, b = rng(1).standard_normal((2, 3001)).astype(np.float32)
    assert np.array_equal(O().elementwise("add", a, b), a + b)
    assert np.array_equal(O().elementwise("mul", a, b), a * b)
    # u * (v + 1): the signal is the first operand, the gate the second.
    assert np.array_equal(O().elementwise("gate_apply", a, b), a * (b + np.float32(1)))
    assert not np.array_equal(O().elementwise("gate_apply", a, b), b * (a + np.float32(1)))


def test_lrelu_relu_and_chan_scale():
    x = rng(2).standard_normal(4097).astype(np.float32)
    assert np.array_equal(O().elementwise("lrelu", x, slope=0.2), np.where(x >= 0, x, np.float32(0.2) * x))
    r = O().elementwise("lrelu", x, slope=0.0)
    assert np.array_equal(r, np.maximum(x, 0)) and (r >= 0).all()
    x3 = rng(3).standard_normal((5, 7, 9)).astype(np.float32)
    s = rng(4).standard_normal(5).astype(np.float32)
    assert np.array_equal(O().chan_scale(x3, s), x3 * s[:, None, None])


def test_gelu_is_the_erf_form():
    x = np.concatenate([np.linspace(-8, 8, 4001), [0.0, -0.0, 1e-30, 30.0]]).astype(np.float32)
    want = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    got = O().elementwise("gelu", x)
    assert np.abs(got - want).max() <= 4e-7 * (1 + np.abs(want)).max()
    # not the tanh approximation
    tanh = 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x.astype(np.float64) ** 3)))
    assert np.abs(got - tanh).max() > 1e-4


def test_sigmoid():
    x = np.linspace(-40, 40, 8001).astype(np.float32)
    want = 1 / (1 + np.exp(-x.astype(np.float64)))
    assert np.abs(O().elementwise("sigmoid", x) - want).max() <= 2e-7


# ------------------------------------------------------------ channel axis

def test_chan_ln_against_float64():
    """Biased variance, eps = 1e-6 inside the square root, scale then bias.

    Pixel (0, 0) has zero mean and a variance (1e-8) far below eps, which is
    where the position of eps shows; pixel (0, 1) is constant (variance 0, so
    y = bias exactly); pixel (0, 2) has mean 3 and the same tiny spread, where
    the reference's one-pass variance s2/c - m^2 cancels in fp32 (kept on
    purpose, src/exec_cpu.rs:403-406) - there only a loose bound holds."""
    x = rng(5).standard_normal((32, 50, 7)).astype(np.float32)
    tiny = np.float32(1e-4) * rng(6).standard_normal(32).astype(np.float32)
    x[:, 0, 0] = tiny
    x[:, 0, 1] = 2.5
    x[:, 0, 2] = np.float32(3.0) + tiny
    s = (1 + 0.1 * rng(7).standard_normal(32)).astype(np.float32)
    b = (0.1 * rng(8).standard_normal(32)).astype(np.float32)
    got = O().chan_ln(x, s, b)
    xd = x.astype(np.float64)
    want = (xd - xd.mean(0)) / np.sqrt(xd.var(0) + 1e-6) * s[:, None, None] + b[:, None, None]
    d = np.abs(got - want)
    d[:, 0, 2] = 0
    assert d.max() <= 1e-5 * np.abs(want).max()
    assert np.array_equal(got[:, 0, 1], b)
    # eps outside the root, or an unbiased variance, would miss this by > 1%:
    wrong = (xd[:, 0, 0] - xd[:, 0, 0].mean()) / (np.sqrt(xd[:, 0, 0].var()) + 1e-6)
    assert np.abs(got[:, 0, 0] - want[:, 0, 0]).max() <= 1e-5
    assert np.abs(wrong * s + b - want[:, 0, 0]).max() > 1e-2
    assert np.abs(got[:, 0, 2] - want[:, 0, 2]).max() <= 0.05


def ln_one_pass_fp32(x, s, b):
    """The reference's LayerNorm in fp32, step by step (src/exec_cpu.rs:392-432):
    ascending s1 = sum x and s2 = sum x^2, m = s1 / c, var = s2 / c - m^2,
    r = 1 / sqrt(max(var, 0) + 1e-6), y = (x - m) * r * w + b."""
    f = np.float32
    c = x.shape[0]
    s1 = np.zeros(x.shape[1:], f)
    s2 = np.zeros(x.shape[1:], f)
    for k in range(c):
        s1 = (s1 + x[k]).astype(f)
        s2 = (s2 + (x[k] * x[k]).astype(f)).astype(f)
    m = (s1 / f(c)).astype(f)
    var = (s2 / f(c) - (m * m).astype(f)).astype(f)
    r = (f(1) / np.sqrt((np.maximum(var, f(0)) + f(1e-6)).astype(f))).astype(f)
    return ((((x - m).astype(f) * r).astype(f) * s[:, None, None]).astype(f) + b[:, None, None]).astype(f)


def ln_variance_case():
    """Pixels where the one-pass fp32 variance and a two-pass one disagree by
    orders of magnitude: a large common offset (1000, 5000) under a spread of
    ~0.05, where s2 / c - m^2 cancels to a few ulps of m^2 (so r is far from
    1 / 0.05), and a plain pixel for contrast."""
    g = rng(31)
    c = 32
    x = np.empty((c, 1, 3), np.float32)
    x[:, 0, 0] = np.float32(1000.0) + (0.05 * g.standard_normal(c)).astype(np.float32)
    x[:, 0, 1] = np.float32(5000.0) + (0.05 * g.standard_normal(c)).astype(np.float32)
    x[:, 0, 2] = g.standard_normal(c).astype(np.float32)
    s = (1 + 0.1 * g.standard_normal(c)).astype(np.float32)
    b = (0.1 * g.standard_normal(c)).astype(np.float32)
    return x, s, b


def test_chan_ln_one_pass_variance_known_answer():
    """The variance is the reference's one-pass s2 / c - m^2 in fp32
    (src/exec_cpu.rs:403-406), not a two-pass sum of squared deviations: on
    pixels where the two differ by orders of magnitude the oracle gives the
    one-pass bits exactly."""
    x, s, b = ln_variance_case()
    got = O().chan_ln(x, s, b)
    want = ln_one_pass_fp32(x, s, b)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the case discriminates: a two-pass variance gives a different answer
    xd = x.astype(np.float64)
    two = (xd - xd.mean(0)) / np.sqrt(xd.var(0) + 1e-6) * s[:, None, None] + b[:, None, None]
    assert np.abs(two[:, 0, :2] - want[:, 0, :2]).max() > 0.5
    assert np.abs(two[:, 0, 2] - want[:, 0, 2]).max() < 1e-4


def test_chan_mean():
    x = rng(9).standard_normal((6, 300, 11)).astype(np.float32) + 2
    assert rel_err(O().chan_mean(x), x.astype(np.float64).mean((1, 2))) <= 1e-6


# ------------------------------------------------------------------ convs

def torch64():
    import torch
    import torch.nn.functional as F
    return torch, F


def test_conv1x1_and_dense():
    x = rng(10).standard_normal((24, 9, 13)).astype(np.float32)
    w = rng(11).standard_normal((40, 24)).astype(np.float32)
    b = rng(12).standard_normal(40).astype(np.float32)
    want = np.einsum("oi,ihw->ohw", w.astype(np.float64), x.astype(np.float64)) + b[:, None, None]
    assert rel_err(O().conv1x1(x, w, b), want) <= 1e-5
    assert rel_err(O().conv1x1(x, w, None), want - b[:, None, None]) <= 1e-5


@pytest.mark.parametrize("ci,co,h,w", [(3, 8, 11, 17), (16, 5, 8, 8), (7, 7, 1, 9)])
def test_conv3x3_pad1_is_torch_conv2d(ci, co, h, w):
    torch, F = torch64()
    x = rng(ci).standard_normal((ci, h, w)).astype(np.float32)
    k = rng(co).standard_normal((co, ci, 3, 3)).astype(np.float32)
    b = rng(h).standard_normal(co).astype(np.float32)
    want = F.conv2d(torch.from_numpy(x).double()[None], torch.from_numpy(k).double(),
                    torch.from_numpy(b).double(), padding=1)[0].numpy()
    assert rel_err(O().conv3x3(x, k, b), want) <= 1e-5


@pytest.mark.parametrize("ci,co,h,w", [(4, 6, 16, 20), (3, 5, 9, 13), (8, 8, 2, 2)])
def test_conv4x4s2_same_is_torch_conv2d(ci, co, h, w):
    """Conv_down: 4x4 stride 2 with flax SAME padding, ceil(h/2) outputs."""
    from maxim_amd import plan as P
    torch, F = torch64()
    x = rng(h).standard_normal((ci, h, w)).astype(np.float32)
    k = rng(w).standard_normal((co, ci, 4, 4)).astype(np.float32)
    b = rng(ci).standard_normal(co).astype(np.float32)
    pt, pb = P.same_pad(h, 2, 4)
    pl, pr = P.same_pad(w, 2, 4)
    xp = F.pad(torch.from_numpy(x).double()[None], (pl, pr, pt, pb))
    want = F.conv2d(xp, torch.from_numpy(k).double(), torch.from_numpy(b).double(), stride=2)[0].numpy()
    got = O().conv4x4s2(x, k, b, pt, pl)
    assert got.shape == want.shape == (co, (h + 1) // 2, (w + 1) // 2)
    assert rel_err(got, want) <= 1e-5


def test_convt2x2_is_torch_conv_transpose2d():
    """The CPU arm scatters with the [ci][co][2][2] weight the loader already
    flipped, which is torch's conv_transpose2d weight (tools/reference.py:90-96)."""
    torch, F = torch64()
    x = rng(13).standard_normal((6, 5, 7)).astype(np.float32)
    k = rng(14).standard_normal((6, 4, 2, 2)).astype(np.float32)
    b = rng(15).standard_normal(4).astype(np.float32)
    want = F.conv_transpose2d(torch.from_numpy(x).double()[None], torch.from_numpy(k).double(),
                              torch.from_numpy(b).double(), stride=2)[0].numpy()
    assert rel_err(O().convt2x2(x, k, b), want) <= 1e-5


@pytest.mark.parametrize("mode", [0, 1])
def test_gate_mm_reduces_the_right_axis(mode):
    c, outer, inner = 3, 12, 10
    x = rng(16).standard_normal((c, outer, inner)).astype(np.float32)
    k = outer if mode == 0 else inner
    w = rng(17).standard_normal((k, k)).astype(np.float32)
    b = rng(18).standard_normal(k).astype(np.float32)
    xd, wd = x.astype(np.float64), w.astype(np.float64)
    if mode == 0:
        want = np.einsum("rt,ctb->crb", wd, xd) + b[None, :, None]
    else:
        want = np.einsum("at,cbt->cba", wd, xd) + b[None, None, :]
    assert rel_err(O().gate_mm(x, w, b, mode), want) <= 1e-5


# ------------------------------------------------------------ index maps

@pytest.mark.parametrize("gh,gw,fh,fw", [(4, 5, 3, 2), (16, 16, 2, 3), (2, 3, 16, 16)])
def test_block_perm_is_the_einops_rearrange(gh, gw, fh, fw):
    """block_images / unblock_images (tools/reference.py:174-188)."""
    c, h, w = 3, gh * fh, gw * fw
    x = rng(19).standard_normal((c, h, w)).astype(np.float32)
    blocked = x.reshape(c, gh, fh, gw, fw).transpose(0, 1, 3, 2, 4).reshape(c, gh * gw, fh * fw)
    got = O().block_perm(x, h, w, gh, gw, fh, fw, forward=True)
    assert np.array_equal(got.reshape(blocked.shape), blocked)
    back = O().block_perm(got, h, w, gh, gw, fh, fw, forward=False)
    assert np.array_equal(back, x)
    swapped = x.reshape(c, gh, fh, gw, fw).transpose(0, 2, 4, 1, 3).reshape(c, fh * fw, gh * gw)
    assert np.array_equal(O().block_perm(x, h, w, gh, gw, fh, fw, swap=True).reshape(swapped.shape), swapped)


@pytest.mark.parametrize("f", [2, 4])
def test_down_s_is_jax_nearest(f):
    """Output i reads input floor((i + 0.5) * f) = f*i + f/2: the ODD samples at 2x."""
    x = rng(20).standard_normal((3, 32, 48)).astype(np.float32)
    got = O().down_s(x, f, f // 2)
    assert np.array_equal(got, x[:, f // 2::f, f // 2::f])
    i = np.arange(32 // f)
    assert np.array_equal(np.floor((i + 0.5) * f).astype(int), f * i + f // 2)


@pytest.mark.parametrize("hin,win,hout,wout", [(32, 40, 8, 10), (32, 40, 16, 20), (8, 10, 32, 40),
                                               (16, 20, 32, 40), (28, 40, 7, 10)])
def test_resize_is_jax_bilinear_with_antialias(hin, win, hout, wout):
    """Against torch's antialiased bilinear (the reference transcription's own
    stand-in for jax.image.resize, tools/reference.py:191-210)."""
    torch, F = torch64()
    x = rng(21).standard_normal((5, hin, win)).astype(np.float32)
    r = hout / hin
    want = F.interpolate(torch.from_numpy(x).double()[None], size=(hout, wout), mode="bilinear",
                         align_corners=False, antialias=r < 1)[0].numpy()
    got = O().resize(x, hout, wout)
    assert rel_err(got, want) <= 1e-5


@pytest.mark.parametrize("n_in,n_out", [(640, 160), (640, 320), (160, 640), (320, 640), (4096, 1024)])
def test_resize_taps(n_in, n_out):
    """The tap table: half-pixel sample positions, a triangle of half-width
    max(n_in/n_out, 1), taps clamped to the row, weights 1 - |s - j| / k."""
    j0, n, s, w = O().resize_taps(n_in, n_out)
    inv = n_in / n_out
    k = max(inv, 1.0)
    for o in range(0, n_out, max(1, n_out // 97)):
        samp = (o + 0.5) * inv - 0.5
        js = [j for j in range(int(math.floor(samp - k)), int(math.ceil(samp + k)) + 1)
              if 0 <= j < n_in and abs(samp - j) / k < 1]
        assert j0[o] == js[0] and n[o] == len(js)
        want = np.array([1 - abs(samp - j) / k for j in js])
        assert np.abs(w[o, :n[o]] - want).max() <= 1e-6
        assert abs(s[o] - want.sum()) <= 1e-5


# ------------------------------------------------------- the whole loop

def test_threads_do_not_change_a_bit():
    """The pool splits work, never a reduction: 1 thread and 8 agree bitwise
    (the identity the reference's MAXIM_SERIAL bisection relies on)."""
    from maxim_amd import plan as P
    plan = P.Plan(weights("S-2"), 64, 64)
    img = rng(22).random((3, 64, 64), dtype=np.float32)
    a = buf(plan, run_oracle(plan, img, threads=1), plan.output).copy()
    b = buf(plan, run_oracle(plan, img, threads=8), plan.output).copy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_memguard():
    """src/memguard.rs:61-172: (arena + 2 * weights + scratch) * 1.05 + 64 MiB."""
    from maxim_amd import plan as P
    plan = P.Plan(weights("S-2"), 256, 256)
    rc, peak, msg = plan.memguard(24, avail=1 << 40)
    assert rc == 0
    scratch = 12 * 24 * (256 * 512 * 4 + 256 * 4 + 128 * 4)  # widest conv1x1: 512 -> 128
    assert peak == int((plan.arena_bytes + 2 * plan.weight_bytes + scratch) * 1.05) + (64 << 20)
    rc, _, msg = plan.memguard(24, avail=100 << 20)
    assert rc != 0 and "not enough memory" in msg and "100 MiB is available" in msg
