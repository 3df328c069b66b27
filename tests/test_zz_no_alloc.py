"""mxh_run_noalloc (no counterpart in the reference): the pass with device
input and output and the code object's static scratch, for callers that
cannot allocate. Checked against mxh_run on the same executor, bit for bit
(the same kernels; only the scratch they use differs), on two calls in a
row, the second with a smaller input; the static scratch keeps the first
call's contents, which every pass overwrites before reading."""

import ctypes as C
import os

import numpy as np
import pytest

from conftest import weights

pytestmark = pytest.mark.gpu


def _hip():
    """The HIP runtime the executor dlopen'd (the same names, in its order),
    for the test's own device buffers: the caller allocates, the entry point
    does not."""
    from maxim_amd import hip as H
    H.driver_ready()  # loads the runtime into the process
    for name in ("libamdhip64.so.7", "libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            rt = C.CDLL(name, mode=os.RTLD_NOLOAD | os.RTLD_GLOBAL)
        except OSError:
            continue
        rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        rt.hipFree.argtypes = [C.c_void_p]
        rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        return rt
    pytest.fail("the HIP runtime is not loaded")


class DevBuf:
    def __init__(self, rt, n):
        self.rt, self.n, self.p = rt, n, C.c_void_p()
        assert rt.hipMalloc(C.byref(self.p), n * 4) == 0

    def put(self, a):
        a = np.ascontiguousarray(a, np.float32).ravel()
        assert a.size == self.n and self.rt.hipMemcpy(self.p, a.ctypes.data, self.n * 4, 1) == 0

    def get(self):
        out = np.empty(self.n, np.float32)
        assert self.rt.hipMemcpy(out.ctypes.data, self.p, self.n * 4, 2) == 0
        return out

    def free(self):
        self.rt.hipFree(self.p)


def _pass(rt, gpu, img):
    c, h, w = gpu.plan.bufs[gpu.plan.output]
    din, dout = DevBuf(rt, img.size), DevBuf(rt, c * h * w)
    try:
        din.put(img)
        dout.put(np.full(c * h * w, np.nan, np.float32))
        gpu.run_noalloc(din.p.value, dout.p.value)
        gpu.sync()
        return dout.get().reshape(c, h, w)
    finally:
        din.free()
        dout.free()


def test_noalloc_matches_run_twice_second_smaller():
    from maxim_amd import hip as H
    from maxim_amd import plan as P
    rt = _hip()
    w = weights("S-2")
    big, small = P.Plan(w, 128, 192), P.Plan(w, 64, 64)
    rng = np.random.default_rng(11)
    for plan in (big, small):
        print("noalloc: S-2 %dx%d" % (plan.shape[1], plan.shape[2]), flush=True)
        img = rng.random(plan.shape, dtype=np.float32)
        g = H.Gpu(plan)
        try:
            ref = g.run(img)
            got = _pass(rt, g, img)
            assert np.array_equal(got, ref), float(np.nanmax(np.abs(got - ref)))
        finally:
            g.close()


def test_noalloc_refuses_a_plan_whose_scratch_does_not_fit():
    """A pass whose scratch exceeds the static array is refused with the
    numbers before anything is launched (mxh_run still runs it)."""
    from maxim_amd import hip as H
    from maxim_amd import plan as P
    plan = P.Plan(weights("S-2"), 2048, 2048)
    g = H.Gpu(plan)
    try:
        with pytest.raises(P.MaximError, match="static scratch"):
            g.run_noalloc(16, 16)
    finally:
        g.close()
