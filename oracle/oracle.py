"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (liboracle.so).

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker; never by the product library.
"""

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError("the oracle is not built (make -C oracle)")
        L = C.CDLL(path)
        P, I, F = C.c_void_p, C.c_int64, C.c_float
        sig = {
            "oracle_run": (C.c_int, [P, P, C.c_int]),
            "oracle_step": (C.c_int, [P, P, C.c_uint64, C.c_int]),
            "oracle_run_range": (C.c_int, [P, P, C.c_uint64, C.c_uint64, C.c_int]),
            "oracle_threads_used": (C.c_int, []),
            "oracle_add": (None, [P, P, P, I]),
            "oracle_mul": (None, [P, P, P, I]),
            "oracle_gate_apply": (None, [P, P, P, I]),
            "oracle_gelu": (None, [P, P, I]),
            "oracle_lrelu": (None, [P, P, I, F]),
            "oracle_sigmoid": (None, [P, P, I]),
            "oracle_chan_ln": (None, [P, P, P, P, I, I]),
            "oracle_chan_mean": (None, [P, P, I, I]),
            "oracle_chan_scale": (None, [P, P, P, I, I]),
            "oracle_conv1x1": (None, [P, P, P, P, I, I, I]),
            "oracle_conv3x3": (None, [P, P, P, P, I, I, I, I]),
            "oracle_conv4x4s2": (None, [P, P, P, P, I, I, I, I, I, I, I, I]),
            "oracle_convt2x2": (None, [P, P, P, P, I, I, I, I]),
            "oracle_gate_mm": (None, [P, P, P, P, I, I, I, C.c_int]),
            "oracle_block_perm": (None, [P, P, I, I, I, I, I, I, I, C.c_int, C.c_int]),
            "oracle_resize": (None, [P, P, P, I, I, I, I, I]),
            "oracle_down_s": (None, [P, P, I, I, I, I, I, I, I]),
            "oracle_resize_taps": (I, [I, I, P, P, P, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def run(plan, arena, threads=0):
    """exec_cpu::run over a maxim_amd.plan.Plan and a float32 arena."""
    assert arena.dtype == np.float32 and arena.size >= plan.arena_len
    rc = lib().oracle_run(C.byref(plan.desc), arena.ctypes.data, threads)
    assert rc == 0, "oracle_run failed"


def run_range(plan, arena, first, last, threads=0):
    rc = lib().oracle_run_range(C.byref(plan.desc), arena.ctypes.data, first, last, threads)
    assert rc == 0


def step(plan, arena, i, threads=0):
    rc = lib().oracle_step(C.byref(plan.desc), arena.ctypes.data, i, threads)
    assert rc == 0


def threads_used():
    return lib().oracle_threads_used()


# ---- the arms on numpy arrays ------------------------------------------------

def elementwise(name, *xs, slope=0.0):
    xs = [_f(x) for x in xs]
    y = np.empty_like(xs[0])
    L = lib()
    if name in ("add", "mul", "gate_apply"):
        getattr(L, "oracle_" + name)(_p(xs[0]), _p(xs[1]), _p(y), y.size)
    elif name == "lrelu":
        L.oracle_lrelu(_p(xs[0]), _p(y), y.size, slope)
    else:
        getattr(L, "oracle_" + name)(_p(xs[0]), _p(y), y.size)
    return y


def chan_ln(x, scale, bias):
    x = _f(x)
    c = x.shape[0]
    y = np.empty_like(x)
    lib().oracle_chan_ln(_p(x), _p(_f(scale)), _p(_f(bias)), _p(y), c, x.size // c)
    return y


def chan_mean(x):
    x = _f(x)
    c = x.shape[0]
    y = np.empty(c, np.float32)
    lib().oracle_chan_mean(_p(x), _p(y), c, x.size // c)
    return y


def chan_scale(x, s):
    x = _f(x)
    c = x.shape[0]
    y = np.empty_like(x)
    lib().oracle_chan_scale(_p(x), _p(_f(s)), _p(y), c, x.size // c)
    return y


def conv1x1(x, w, b):
    """x [ci][h][w], w [co][ci], b [co] or None."""
    x, w = _f(x), _f(w)
    co, ci = w.shape
    y = np.empty((co,) + x.shape[1:], np.float32)
    lib().oracle_conv1x1(_p(x), _p(w), _p(None if b is None else _f(b)), _p(y), ci, co, x[0].size)
    return y


def conv3x3(x, w, b):
    """x [ci][h][w], w [co][ci][3][3]."""
    x, w = _f(x), _f(w)
    co, ci = w.shape[:2]
    _, h, wd = x.shape
    y = np.empty((co, h, wd), np.float32)
    lib().oracle_conv3x3(_p(x), _p(w), _p(None if b is None else _f(b)), _p(y), ci, co, h, wd)
    return y


def conv4x4s2(x, w, b, pad_top, pad_left):
    x, w = _f(x), _f(w)
    co, ci = w.shape[:2]
    _, h, wd = x.shape
    oh, ow = (h + 1) // 2, (wd + 1) // 2
    y = np.empty((co, oh, ow), np.float32)
    lib().oracle_conv4x4s2(_p(x), _p(w), _p(None if b is None else _f(b)), _p(y), ci, co, h, wd,
                           pad_top, pad_left, oh, ow)
    return y


def convt2x2(x, w, b):
    """w [ci][co][2][2], already spatially flipped."""
    x, w = _f(x), _f(w)
    ci, co = w.shape[:2]
    _, h, wd = x.shape
    y = np.empty((co, 2 * h, 2 * wd), np.float32)
    lib().oracle_convt2x2(_p(x), _p(w), _p(None if b is None else _f(b)), _p(y), ci, co, h, wd)
    return y


def gate_mm(x, w, b, mode):
    """x [c][outer][inner]; w [k][k] (output-major); mode 0 reduces outer, 1 inner."""
    x, w = _f(x), _f(w)
    c, outer, inner = x.shape
    y = np.empty_like(x)
    lib().oracle_gate_mm(_p(x), _p(w), _p(None if b is None else _f(b)), _p(y), c, outer, inner, mode)
    return y


def block_perm(x, h, wd, gh, gw, fh, fw, swap=False, forward=True):
    x = _f(x)
    c = x.shape[0]
    y = np.empty_like(x)
    lib().oracle_block_perm(_p(x), _p(y), c, h, wd, gh, gw, fh, fw, int(swap), int(forward))
    return y


def resize(x, hout, wout):
    x = _f(x)
    c, hin, win = x.shape
    tmp = np.empty((c, hin, wout), np.float32)
    y = np.empty((c, hout, wout), np.float32)
    lib().oracle_resize(_p(x), _p(tmp), _p(y), c, hin, win, hout, wout)
    return y


def resize_taps(n_in, n_out):
    j = np.empty(2 * n_out, np.int32)
    s = np.empty(n_out, np.float32)
    w = np.zeros(64 * n_out, np.float32)
    lib().oracle_resize_taps(n_in, n_out, _p(j), _p(j[n_out:]), _p(s), _p(w))
    return j[:n_out], j[n_out:], s, w.reshape(n_out, 64)


def down_s(x, stride, off):
    x = _f(x)
    c, h, wd = x.shape
    oh, ow = h // stride, wd // stride
    y = np.empty((c, oh, ow), np.float32)
    lib().oracle_down_s(_p(x), _p(y), c, h, wd, stride, off, oh, ow)
    return y
