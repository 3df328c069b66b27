"""ctypes binding of the gfx950 executor (include/maxim_hip.h).

`Gpu` mirrors the reference's `exec_gpu::Gpu` (src/exec_gpu.rs:48-357): built
for one plan, it owns the device arena and the device weights; `run` takes an
input image and returns the output image. There is no CPU fallback here: if
the library or the device is missing, the call raises.
"""

import ctypes as C

import numpy as np

from . import plan as P

_declared = False


def _lib():
    global _declared
    L = P.lib()
    if not hasattr(L, "mxh_new"):
        raise P.MaximError("libmaxim_hip.so is not built: the HIP executor is unavailable")
    if not _declared:
        V, U, I = C.c_void_p, C.c_uint64, C.c_int
        D = C.POINTER(P.PlanDesc)
        sig = {
            "mxh_driver_ready": (I, []),
            "mxh_new": (V, [D]),
            "mxh_free": (None, [V]),
            "mxh_run": (I, [V, D, V, U, V, U]),
            "mxh_begin": (I, [V, D, V, U]),
            "mxh_step_op": (I, [V, D, U]),
            "mxh_run_ops": (I, [V, D, U, U]),
            "mxh_read_buf": (I, [V, D, U, V, U]),
            "mxh_read_into": (I, [V, U, V, U]),
            "mxh_read_arena": (I, [V, V, U]),
            "mxh_write_into": (I, [V, U, V, U]),
            "mxh_write_buf": (I, [V, D, U, V, U]),
            "mxh_buf_offset": (U, [V, U]),
            "mxh_poison": (I, [V]),
            "mxh_sync": (I, [V]),
            "mxh_set_timeline": (None, [V, I]),
            "mxh_timeline": (I, [V, V, U, C.POINTER(C.c_float)]),
            "mxh_run_timed": (I, [V, D]),
            "mxh_run_graph": (I, [V, D]),
            "mxh_set_graph": (None, [V, I]),
            "mxh_set_fusion": (None, [V, I]),
            "mxh_fused_ops": (U, [V]),
            "mxh_steps": (U, [V]),
            "mxh_step_info": (I, [V, U, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                  C.POINTER(C.c_char_p)]),
            "mxh_time_ops": (I, [V, D, U, U, I, C.POINTER(C.c_float)]),
            "mxh_launches": (U, [V]),
            "mxh_launch_info": (I, [V, U, C.POINTER(C.c_uint64), C.POINTER(C.c_char_p)]),
            "mxh_launch_span": (I, [V, U, C.POINTER(U)]),
            "mxh_launch_timeline": (I, [V, V, U]),
            "mxh_device_name": (C.c_char_p, [V]),
            "mxh_arena_bytes": (U, [V]),
            "mxh_weight_bytes": (U, [V]),
            "mxh_pool_bytes": (U, [V]),
            "mxh_ops_launched": (U, [V]),
            "mxh_kernels_launched": (U, [V]),
            "mxh_op_kernel": (C.c_char_p, [V, U]),
            "mxh_device_info": (I, [V, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
            "mxh_device_memory": (I, [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
            "mxh_run_noalloc": (I, [V, D, V, U, V, U, V]),
            "mxh_run_batch": (I, [V, D, C.POINTER(V), U, C.POINTER(V), U, U]),
            "mxh_time_graph": (I, [V, D, C.c_int, V]),
            "mxh_enhance": (I, [C.c_char_p, V, C.c_int64, C.c_int64, V]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _declared = True
    return L


def _check(rc):
    if rc != 0:
        raise P.MaximError(P.last_error())


def device_memory():
    """(free, total) bytes of device 0."""
    f, t = C.c_uint64(), C.c_uint64()
    _check(_lib().mxh_device_memory(C.byref(f), C.byref(t)))
    return f.value, t.value


def enhance(checkpoint, image):
    """mxh_enhance: checkpoint file + [3][h][w] image -> the cropped
    prediction (the reference's run with the HIP backend)."""
    img = np.ascontiguousarray(image, np.float32)
    out = np.empty_like(img)
    _check(_lib().mxh_enhance(checkpoint.encode(), img.ctypes.data, img.shape[1], img.shape[2], out.ctypes.data))
    return out


def driver_ready():
    """exec_gpu::driver_ready: True when the HIP runtime and a device come up."""
    return _lib().mxh_driver_ready() == 0


class Gpu:
    def __init__(self, plan):
        L = _lib()
        self.plan = plan
        self._d = C.byref(plan.desc)
        self._h = L.mxh_new(self._d)
        if not self._h:
            raise P.MaximError(P.last_error())

    def close(self):
        if getattr(self, "_h", None):
            _lib().mxh_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run(self, image):
        img = np.ascontiguousarray(image, dtype=np.float32)
        c, h, w = self.plan.bufs[self.plan.output]
        out = np.empty((c, h, w), np.float32)
        _check(_lib().mxh_run(self._h, self._d, img.ctypes.data, img.size, out.ctypes.data, out.size))
        return out

    def run_batch(self, images):
        """mxh_run_batch: every image of the list through the pass, the
        host's staging overlapped with the passes; the outputs, each
        mxh_run's to the bit."""
        imgs = [np.ascontiguousarray(im, dtype=np.float32) for im in images]
        c, h, w = self.plan.bufs[self.plan.output]
        outs = [np.empty((c, h, w), np.float32) for _ in imgs]
        n_in = int(np.prod(self.plan.bufs[self.plan.input]))
        for im in imgs:
            if im.size != n_in:
                raise P.MaximError("the input image and the plan's input buffer disagree")
        ins = (C.c_void_p * max(len(imgs), 1))(*[im.ctypes.data for im in imgs])
        ous = (C.c_void_p * max(len(outs), 1))(*[o.ctypes.data for o in outs])
        _check(_lib().mxh_run_batch(self._h, self._d, ins, n_in, ous, c * h * w, len(imgs)))
        return outs

    def run_noalloc(self, d_input, d_output, stream=None):
        """mxh_run_noalloc: the pass from device pointer d_input to d_output
        (integers), asynchronously on `stream` (a hipStream_t as an integer;
        None: the executor's stream), with no allocation (the static
        scratch)."""
        c, h, w = self.plan.bufs[self.plan.input]
        co, ho, wo = self.plan.bufs[self.plan.output]
        _check(_lib().mxh_run_noalloc(self._h, self._d, d_input, c * h * w, d_output, co * ho * wo, stream))

    def begin(self, image):
        img = np.ascontiguousarray(image, dtype=np.float32)
        _check(_lib().mxh_begin(self._h, self._d, img.ctypes.data, img.size))

    def step_op(self, i):
        _check(_lib().mxh_step_op(self._h, self._d, i))

    def run_ops(self, first, last):
        _check(_lib().mxh_run_ops(self._h, self._d, first, last))

    def read_buf(self, buf):
        n = self.plan.buf_len(buf)
        out = np.empty(n, np.float32)
        _check(_lib().mxh_read_buf(self._h, self._d, buf, out.ctypes.data, n))
        return out

    def read_into(self, off, n):
        out = np.empty(n, np.float32)
        _check(_lib().mxh_read_into(self._h, off, out.ctypes.data, n))
        return out

    def write_into(self, off, data):
        d = np.ascontiguousarray(data, dtype=np.float32)
        _check(_lib().mxh_write_into(self._h, off, d.ctypes.data, d.size))

    def write_buf(self, buf, data):
        d = np.ascontiguousarray(data, dtype=np.float32)
        _check(_lib().mxh_write_buf(self._h, self._d, buf, d.ctypes.data, d.size))

    def buf_offset(self, buf):
        """Where buffer `buf` lives in the device arena (elements)."""
        return _lib().mxh_buf_offset(self._h, buf)

    def read_arena(self):
        out = np.empty(self.arena_bytes // 4, np.float32)
        _check(_lib().mxh_read_arena(self._h, out.ctypes.data, out.size))
        return out

    def poison(self):
        _check(_lib().mxh_poison(self._h))

    def sync(self):
        _check(_lib().mxh_sync(self._h))

    def set_timeline(self, on=True):
        _lib().mxh_set_timeline(self._h, int(on))

    def set_fusion(self, on=True):
        _lib().mxh_set_fusion(self._h, int(on))

    @property
    def fused_ops(self):
        return _lib().mxh_fused_ops(self._h)

    def steps(self):
        """[(first op, last op + 1, kernel)] of the program mxh_run executes."""
        L = _lib()
        out = []
        a, b, k = C.c_uint64(), C.c_uint64(), C.c_char_p()
        for i in range(L.mxh_steps(self._h)):
            _check(L.mxh_step_info(self._h, i, C.byref(a), C.byref(b), C.byref(k)))
            out.append((a.value, b.value, k.value.decode()))
        return out

    def timeline(self):
        n = _lib().mxh_steps(self._h)
        per = np.empty(n, np.float32)
        tot = C.c_float()
        _check(_lib().mxh_timeline(self._h, per.ctypes.data, n, C.byref(tot)))
        return per, tot.value

    def run_graph(self):
        """Every op over the resident input as one graph replay (asynchronous)."""
        _check(_lib().mxh_run_graph(self._h, self._d))

    def set_graph(self, on=True):
        _lib().mxh_set_graph(self._h, int(on))

    def run_timed(self):
        """Every step over the resident input, one event per step: (per-step ms, total ms)."""
        _check(_lib().mxh_run_timed(self._h, self._d))
        return self.timeline()

    def launches(self):
        """[(step, kernel)] of every launch of the current program, in order."""
        L = _lib()
        out = []
        st, k = C.c_uint64(), C.c_char_p()
        for i in range(L.mxh_launches(self._h)):
            _check(L.mxh_launch_info(self._h, i, C.byref(st), C.byref(k)))
            out.append((st.value, k.value.decode()))
        return out

    def launch_spans(self):
        """[((first, last), (first2, last2) or None)] - the ops each launch
        computes (a second range for a launch pairing two steps' work)."""
        L = _lib()
        out = []
        o = (C.c_uint64 * 4)()
        for i in range(L.mxh_launches(self._h)):
            _check(L.mxh_launch_span(self._h, i, o))
            out.append(((o[0], o[1]), (o[2], o[3]) if o[3] > o[2] else None))
        return out

    def launch_timeline(self):
        """Per-launch device ms of the last run_timed()."""
        n = _lib().mxh_launches(self._h)
        ms = np.empty(n, np.float32)
        _check(_lib().mxh_launch_timeline(self._h, ms.ctypes.data, n))
        return ms

    def time_graph(self, n):
        """n graph replays back to back, each bracketed by its own events:
        per-pass device ms."""
        ms = np.empty(n, np.float32)
        _check(_lib().mxh_time_graph(self._h, self._d, n, ms.ctypes.data))
        return ms

    def time_ops(self, first, last, iters=1):
        ms = C.c_float()
        _check(_lib().mxh_time_ops(self._h, self._d, first, last, iters, C.byref(ms)))
        return ms.value

    def op_kernel(self, i):
        return _lib().mxh_op_kernel(self._h, i).decode()

    @property
    def device_name(self):
        return _lib().mxh_device_name(self._h).decode()

    @property
    def arena_bytes(self):
        return _lib().mxh_arena_bytes(self._h)

    @property
    def weight_bytes(self):
        return _lib().mxh_weight_bytes(self._h)

    @property
    def pool_bytes(self):
        return _lib().mxh_pool_bytes(self._h)

    @property
    def ops_launched(self):
        return _lib().mxh_ops_launched(self._h)

    @property
    def kernels_launched(self):
        return _lib().mxh_kernels_launched(self._h)

    def device_info(self):
        cu, clk = C.c_int(), C.c_int()
        _lib().mxh_device_info(self._h, C.byref(cu), C.byref(clk))
        return cu.value, clk.value
