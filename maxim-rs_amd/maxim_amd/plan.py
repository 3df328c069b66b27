"""ctypes binding of the plan contract (include/maxim_plan.h).

The plan is built by the C++ host library; this module only marshals it so
that tests and the benchmark can read the op list, the buffer table and the
arena offsets, and hand the same plan to an executor.
"""

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# MAXIM_LIB_DIR: another build of the libraries (e.g. lib-san, the host
# code under the address and undefined-behaviour sanitizers)
LIB_DIR = os.environ.get("MAXIM_LIB_DIR") or os.path.join(os.path.dirname(_HERE), "lib")

OP_NAMES = [
    "copy", "add", "mul", "gate_apply", "gelu", "lrelu", "sigmoid", "chan_ln",
    "chan_mean", "chan_scale", "conv1x1", "conv3x3", "conv4x4s2", "convt2x2",
    "gate_mm", "block_perm", "resize", "down_s",
]
(COPY, ADD, MUL, GATE_APPLY, GELU, LRELU, SIGMOID, CHAN_LN, CHAN_MEAN, CHAN_SCALE,
 CONV1X1, CONV3X3, CONV4X4S2, CONVT2X2, GATE_MM, BLOCK_PERM, RESIZE, DOWN_S) = range(18)
PERM_SWAP, PERM_FORWARD = 1, 2


class Op(C.Structure):
    _fields_ = [
        ("kind", C.c_int32), ("mode", C.c_int32), ("slope", C.c_float), ("reserved", C.c_int32),
        ("dst", C.c_int64), ("src", C.c_int64), ("src2", C.c_int64),
        ("w", C.c_int64), ("wt", C.c_int64), ("bias", C.c_int64), ("scale", C.c_int64),
        ("n", C.c_int64), ("c", C.c_int64), ("hw", C.c_int64),
        ("c_in", C.c_int64), ("c_out", C.c_int64), ("h", C.c_int64), ("wd", C.c_int64),
        ("oh", C.c_int64), ("ow", C.c_int64), ("p", C.c_int64 * 4),
    ]

    def describe(self):
        k = self.kind
        if k in (CONV1X1, CONV3X3, CONV4X4S2, CONVT2X2):
            return "%s %d->%d @%dx%d" % (OP_NAMES[k], self.c_in, self.c_out, self.h, self.wd)
        if k == GATE_MM:
            return "gate_mm c=%d %dx%d mode%d" % (self.c, self.p[0], self.p[1], self.mode)
        if k == BLOCK_PERM:
            return "block_perm %dx%d %dx%d %s" % (self.p[0], self.p[1], self.p[2], self.p[3],
                                                  "in" if self.mode & PERM_FORWARD else "out")
        if k == RESIZE:
            return "resize c=%d %dx%d->%dx%d" % (self.c, self.h, self.wd, self.oh, self.ow)
        if k in (CHAN_LN, CHAN_MEAN, CHAN_SCALE):
            return "%s %dx%d" % (OP_NAMES[k], self.c, self.hw)
        if k == DOWN_S:
            return "down_s stride%d off%d" % (self.p[0], self.p[1])
        return "%s %d" % (OP_NAMES[k], self.n)


class BufShape(C.Structure):
    _fields_ = [("c", C.c_int64), ("h", C.c_int64), ("w", C.c_int64)]


class PlanDesc(C.Structure):
    _fields_ = [
        ("n_ops", C.c_uint64), ("ops", C.POINTER(Op)),
        ("n_bufs", C.c_uint64), ("bufs", C.POINTER(BufShape)), ("offs", C.POINTER(C.c_uint64)),
        ("n_weights", C.c_uint64), ("weights", C.POINTER(C.POINTER(C.c_float))),
        ("weight_lens", C.POINTER(C.c_uint64)),
        ("arena_len", C.c_uint64), ("input", C.c_uint64), ("output", C.c_uint64),
        ("alias_parent", C.POINTER(C.c_int64)), ("alias_delta", C.POINTER(C.c_uint64)),
        ("keep", C.POINTER(C.c_uint8)),
    ]


class Config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "features", "depth", "num_stages", "num_groups", "num_supervision_scales", "num_outputs",
        "use_cross_gating", "high_res_stages", "block_size_hr", "block_size_lr", "grid_size_hr",
        "grid_size_lr", "channels_reduction", "num_bottleneck_blocks")]


class MaximError(RuntimeError):
    """The library's error string (the reference's `maxim::Error`)."""


_lib = None


def _declare(lib):
    P, V = C.c_void_p, None
    sig = {
        "mx_last_error": (C.c_char_p, []),
        "mx_config_variant": (C.c_int, [C.c_char_p, C.POINTER(Config)]),
        "mx_config_for_task": (C.c_int, [C.c_char_p, C.POINTER(Config)]),
        "mx_weights_open": (P, [C.c_char_p]),
        "mx_weights_synthetic": (P, [C.c_char_p, C.c_uint64, C.c_float, C.c_float, C.c_float]),
        "mx_weights_save": (C.c_int, [P, C.c_char_p, C.c_char_p]),
        "mx_weights_config": (C.c_int, [P, C.POINTER(Config)]),
        "mx_weights_count": (C.c_uint64, [P]),
        "mx_weights_params": (C.c_uint64, [P]),
        "mx_weights_name": (C.c_char_p, [P, C.c_uint64]),
        "mx_weights_tensor": (C.c_uint64, [P, C.c_char_p, C.POINTER(C.POINTER(C.c_float)),
                                           C.POINTER(C.c_int64), C.POINTER(C.c_int32)]),
        "mx_weights_free": (V, [P]),
        "mx_plan_build": (P, [P, C.c_int64, C.c_int64, C.c_int, C.c_int, C.c_int]),
        "mx_plan_free": (V, [P]),
        "mx_plan_describe": (V, [P, C.POINTER(PlanDesc)]),
        "mx_plan_n_dumps": (C.c_uint64, [P]),
        "mx_plan_dump_name": (C.c_char_p, [P, C.c_uint64]),
        "mx_plan_dump_buf": (C.c_int64, [P, C.c_uint64]),
        "mx_plan_label": (C.c_char_p, [P, C.c_uint64]),
        "mx_plan_alias_parent": (C.c_int64, [P, C.c_uint64]),
        "mx_plan_alias_delta": (C.c_uint64, [P, C.c_uint64]),
        "mx_plan_weight_bytes": (C.c_uint64, [P]),
        "mx_same_pad": (V, [C.c_int64, C.c_int64, C.c_int64, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "mx_preprocess": (C.c_int, [P, C.c_int64, C.c_int64, C.c_int64, C.c_int64, P,
                                    C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                    C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "mx_crop_out": (C.c_int, [P, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64,
                                  C.c_int64, C.c_int64, P]),
        "mx_memguard_check": (C.c_int, [P, C.c_int, C.c_int64, C.POINTER(C.c_uint64)]),
        "mx_png_open": (C.c_int, [C.c_char_p, P, C.c_size_t, C.POINTER(C.c_void_p), C.POINTER(C.c_int64),
                                  C.POINTER(C.c_int64)]),
        "mx_png_pixels": (C.c_int, [C.c_void_p, P, C.c_size_t]),
        "mx_png_close": (None, [C.c_void_p]),
        "mx_png_encode": (C.c_int, [P, C.c_int64, C.c_int64, P, C.c_size_t, C.POINTER(C.c_size_t)]),
        "mx_png_write": (C.c_int, [C.c_char_p, P, C.c_int64, C.c_int64]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


def lib():
    """The product library when it is built, else the plan-only one."""
    global _lib
    if _lib is None:
        for name in ("libmaxim_hip.so", "libmaxim_plan.so"):
            path = os.path.join(LIB_DIR, name)
            if os.path.exists(path):
                _lib = _declare(C.CDLL(path))
                break
        else:
            raise MaximError("the maxim library is not built (run __graft_entry__.build())")
    return _lib


def last_error():
    return lib().mx_last_error().decode()


def _check(rc):
    if rc != 0:
        raise MaximError(last_error())


def config(variant):
    c = Config()
    _check(lib().mx_config_variant(variant.encode(), C.byref(c)))
    return c


class Weights:
    """A checkpoint: a safetensors file or seeded random-init weights."""

    def __init__(self, handle):
        if not handle:
            raise MaximError(last_error())
        self._h = handle

    @classmethod
    def open(cls, path):
        return cls(lib().mx_weights_open(path.encode()))

    @classmethod
    def synthetic(cls, variant="S-2", seed=0, gain=1.0, bias_std=0.0, ln_std=0.0):
        return cls(lib().mx_weights_synthetic(variant.encode(), seed, gain, bias_std, ln_std))

    def save(self, path, task="enhancement"):
        _check(lib().mx_weights_save(self._h, path.encode(), task.encode()))

    @property
    def config(self):
        c = Config()
        lib().mx_weights_config(self._h, C.byref(c))
        return c

    @property
    def count(self):
        return lib().mx_weights_count(self._h)

    @property
    def params(self):
        return lib().mx_weights_params(self._h)

    def names(self):
        L = lib()
        return [L.mx_weights_name(self._h, i).decode() for i in range(self.count)]

    def flat(self):
        """Every tensor, Flax layout, as a name -> ndarray dict."""
        return {n: self.tensor(n) for n in self.names()}

    def tensor(self, name):
        data = C.POINTER(C.c_float)()
        shape = (C.c_int64 * 4)()
        nd = C.c_int32()
        n = lib().mx_weights_tensor(self._h, name.encode(), C.byref(data), shape, C.byref(nd))
        if n == 0:
            raise KeyError(name)
        return np.ctypeslib.as_array(data, shape=(n,)).reshape(tuple(shape[:nd.value])).copy()

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.mx_weights_free(self._h)
            self._h = None


class Plan:
    """A built plan: ops, buffers, packed offsets and weight blobs."""

    def __init__(self, weights, h, w, named=False, gpu_twins=True, deep=False):
        self.weights_ref = weights
        self._h = lib().mx_plan_build(weights._h, h, w, int(named), int(gpu_twins), int(deep))
        if not self._h:
            raise MaximError(last_error())
        self.desc = PlanDesc()
        lib().mx_plan_describe(self._h, C.byref(self.desc))
        d = self.desc
        self.ops = [d.ops[i] for i in range(d.n_ops)]
        self.bufs = [(d.bufs[i].c, d.bufs[i].h, d.bufs[i].w) for i in range(d.n_bufs)]
        self.offs = np.ctypeslib.as_array(d.offs, shape=(d.n_bufs,)).copy()
        self.arena_len = d.arena_len
        self.input = d.input
        self.output = d.output
        self.shape = (3, h, w)

    @property
    def n_weights(self):
        return self.desc.n_weights

    def weight(self, i):
        n = self.desc.weight_lens[i]
        return np.ctypeslib.as_array(self.desc.weights[i], shape=(n,))

    @property
    def weight_bytes(self):
        return lib().mx_plan_weight_bytes(self._h)

    @property
    def arena_bytes(self):
        return self.arena_len * 4

    def buf_len(self, i):
        c, h, w = self.bufs[i]
        return c * h * w

    def label(self, i):
        return lib().mx_plan_label(self._h, i).decode()

    def alias(self, i):
        p = lib().mx_plan_alias_parent(self._h, i)
        return None if p < 0 else (p, lib().mx_plan_alias_delta(self._h, i))

    @property
    def dumps(self):
        L = lib()
        return [(L.mx_plan_dump_name(self._h, i).decode(), L.mx_plan_dump_buf(self._h, i))
                for i in range(L.mx_plan_n_dumps(self._h))]

    def operands(self, op):
        if op.kind in (ADD, MUL, GATE_APPLY, CHAN_SCALE, RESIZE):
            return [op.dst, op.src, op.src2]
        return [op.dst, op.src]

    def memguard(self, threads, avail=-1):
        peak = C.c_uint64()
        rc = lib().mx_memguard_check(self._h, threads, avail, C.byref(peak))
        return rc, peak.value, (last_error() if rc else "")

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.mx_plan_free(self._h)
            self._h = None


def same_pad(size, stride, k):
    a, b = C.c_int64(), C.c_int64()
    lib().mx_same_pad(size, stride, k, C.byref(a), C.byref(b))
    return a.value, b.value


class Padded:
    def __init__(self, img, orig_h, orig_w, even_h, even_w):
        self.img, self.orig_h, self.orig_w, self.even_h, self.even_w = img, orig_h, orig_w, even_h, even_w


def preprocess(img, factor=64):
    """image::preprocess: even-ize then centred reflect pad to a multiple of `factor`."""
    img = np.ascontiguousarray(img, dtype=np.float32)
    c, h, w = img.shape
    ph, pw, eh, ew = C.c_int64(), C.c_int64(), C.c_int64(), C.c_int64()
    L = lib()
    _check(L.mx_preprocess(img.ctypes.data, c, h, w, factor, None, C.byref(ph), C.byref(pw),
                           C.byref(eh), C.byref(ew)))
    out = np.empty((c, ph.value, pw.value), np.float32)
    _check(L.mx_preprocess(img.ctypes.data, c, h, w, factor, out.ctypes.data, C.byref(ph),
                           C.byref(pw), C.byref(eh), C.byref(ew)))
    return Padded(out, h, w, eh.value, ew.value)


def crop_out(img, p):
    img = np.ascontiguousarray(img, dtype=np.float32)
    c, ph, pw = img.shape
    out = np.empty((c, p.orig_h, p.orig_w), np.float32)
    _check(lib().mx_crop_out(img.ctypes.data, c, ph, pw, p.even_h, p.even_w, p.orig_h, p.orig_w,
                             out.ctypes.data))
    return out


def make_op(kind, **kw):
    """An Op with every index field at -1 unless given."""
    o = Op()
    o.kind = kind
    for f in ("dst", "src", "src2", "w", "wt", "bias", "scale"):
        setattr(o, f, -1)
    for k, v in kw.items():
        if k == "p":
            for i, x in enumerate(v):
                o.p[i] = x
        else:
            setattr(o, k, v)
    return o


class CustomPlan:
    """A plan assembled by hand: buffers packed back to back, one op list.

    This is what any host that owns its own plan does at the boundary: fill an
    mx_plan_desc from its own arrays. Used for the isolated-op configurations.
    `views` = {buffer: (parent, delta)} makes a buffer a view of an earlier
    one (at `delta` elements into it) and hands the executor the view table,
    so it lays out its own device arena as it does for a built plan.
    """

    def __init__(self, bufs, ops, weights, input=0, output=None, align=64, views=None):
        self.bufs = [tuple(int(v) for v in b) for b in bufs]
        views = views or {}
        offs, off = [], 0
        for i, (c, h, w) in enumerate(self.bufs):
            if i in views:
                par, delta = views[i]
                assert par < i and delta + c * h * w <= self.buf_len_of(par), "a view inside an earlier buffer"
                offs.append(offs[par] + delta)
                continue
            offs.append(off)
            off += c * h * w
            off = (off + align - 1) // align * align
        self.offs = np.array(offs, np.uint64)
        self.arena_len = max(off, 1)
        self.ops = list(ops)
        self.input = input
        self.output = output if output is not None else ops[-1].dst
        self._weights = [np.ascontiguousarray(w, dtype=np.float32).ravel() for w in weights]
        self._ops = (Op * max(len(ops), 1))(*ops)
        self._bufs = (BufShape * len(bufs))(*[BufShape(*b) for b in self.bufs])
        self._offs = (C.c_uint64 * len(offs))(*[int(x) for x in offs])
        nw = max(len(self._weights), 1)
        self._wptr = (C.POINTER(C.c_float) * nw)(*[w.ctypes.data_as(C.POINTER(C.c_float)) for w in self._weights])
        self._wlen = (C.c_uint64 * nw)(*[w.size for w in self._weights])
        d = PlanDesc()
        d.n_ops, d.ops = len(ops), self._ops
        d.n_bufs, d.bufs, d.offs = len(bufs), self._bufs, self._offs
        d.n_weights, d.weights, d.weight_lens = len(self._weights), self._wptr, self._wlen
        d.arena_len, d.input, d.output = self.arena_len, self.input, self.output
        if views:
            nb = len(self.bufs)
            self._apar = (C.c_int64 * nb)(*[views[i][0] if i in views else -1 for i in range(nb)])
            self._adel = (C.c_uint64 * nb)(*[views[i][1] if i in views else 0 for i in range(nb)])
            d.alias_parent, d.alias_delta = self._apar, self._adel
        self.desc = d
        self.shape = self.bufs[self.input]

    def buf_len_of(self, i):
        c, h, w = self.bufs[i]
        return c * h * w

    def buf_len(self, i):
        c, h, w = self.bufs[i]
        return c * h * w

    def weight(self, i):
        return self._weights[i]


def read_png(path=None, data=None):
    """image::read_png / read_png_stream: an 8-bit PNG (plain or Adam7
    interlaced), from the file `path` or the bytes `data`, as a [3][h][w]
    float32 array in 0..1; decoded once."""
    h, w, img = C.c_int64(), C.c_int64(), C.c_void_p()
    if path is not None:
        _check(lib().mx_png_open(path.encode(), None, 0, C.byref(img), C.byref(h), C.byref(w)))
    else:
        buf = (C.c_ubyte * len(data)).from_buffer_copy(data)
        _check(lib().mx_png_open(None, C.cast(buf, C.c_void_p), len(data), C.byref(img), C.byref(h), C.byref(w)))
    try:
        out = np.empty((3, h.value, w.value), np.float32)
        _check(lib().mx_png_pixels(img, out.ctypes.data, out.size))
    finally:
        lib().mx_png_close(img)
    return out


def encode_png(img):
    """image::write_png_stream into memory: [3][h][w] in 0..1 as PNG bytes."""
    a = np.ascontiguousarray(img, np.float32)
    assert a.ndim == 3 and a.shape[0] == 3, a.shape
    n = C.c_size_t()
    _check(lib().mx_png_encode(a.ctypes.data, a.shape[1], a.shape[2], None, 0, C.byref(n)))
    out = (C.c_ubyte * n.value)()
    _check(lib().mx_png_encode(a.ctypes.data, a.shape[1], a.shape[2], C.cast(out, C.c_void_p), n.value, C.byref(n)))
    return bytes(out)


def write_png(path, img):
    """image::write_png: [3][h][w] in 0..1 as an 8-bit RGB PNG."""
    a = np.ascontiguousarray(img, np.float32)
    assert a.ndim == 3 and a.shape[0] == 3, a.shape
    _check(lib().mx_png_write(path.encode(), a.ctypes.data, a.shape[1], a.shape[2]))
