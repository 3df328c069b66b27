"""mxh_run_noalloc (no counterpart in the reference): the pass with device
input and output and the code object's static scratch, for callers that
cannot allocate. Checked against mxh_run on the same executor, bit for bit
(the same kernels; only the scratch they use differs), on two calls in a
row, the second with a smaller input; the static scratch keeps the first
call's contents, which every pass overwrites before reading. Also at the
headline size (MAXIM-3S 640x448, whose scratch must fit the static array),
on a stream of the caller's, and captured by the caller into a HIP graph
(global capture mode, which refuses an allocation inside the capture)."""

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
        rt.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        rt.hipStreamDestroy.argtypes = [C.c_void_p]
        rt.hipStreamSynchronize.argtypes = [C.c_void_p]
        rt.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        rt.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        rt.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
        rt.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        rt.hipGraphExecDestroy.argtypes = [C.c_void_p]
        rt.hipGraphDestroy.argtypes = [C.c_void_p]
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


def _pass(rt, gpu, img, stream=None):
    c, h, w = gpu.plan.bufs[gpu.plan.output]
    din, dout = DevBuf(rt, img.size), DevBuf(rt, c * h * w)
    try:
        din.put(img)
        dout.put(np.full(c * h * w, np.nan, np.float32))
        gpu.run_noalloc(din.p.value, dout.p.value, stream)
        if stream is None:
            gpu.sync()
        else:
            assert rt.hipStreamSynchronize(stream) == 0
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


def test_noalloc_at_the_headline_size():
    """MAXIM-3S at 640x448 (the benchmark's configuration) runs through the
    static scratch and equals mxh_run bit for bit."""
    from maxim_amd import hip as H
    from maxim_amd import plan as P
    from conftest import smooth_image
    rt = _hip()
    pad = P.preprocess(smooth_image(400, 600, seed=4), 64)
    plan = P.Plan(weights("S-3"), *pad.img.shape[1:])
    print("noalloc: S-3 %dx%d" % (plan.shape[1], plan.shape[2]), flush=True)
    g = H.Gpu(plan)
    try:
        ref = g.run(pad.img)
        got = _pass(rt, g, pad.img)
        assert np.array_equal(got, ref), float(np.nanmax(np.abs(got - ref)))
    finally:
        g.close()


def test_noalloc_on_a_caller_stream_and_under_capture():
    """The pass queued on the caller's stream, then captured by the caller
    (global mode) and replayed three times, each replay checked against the
    eager mxh_run pass, with eager passes of the executor in between."""
    from maxim_amd import hip as H
    from maxim_amd import plan as P
    rt = _hip()
    plan = P.Plan(weights("S-2"), 128, 128)
    rng = np.random.default_rng(12)
    img = rng.random(plan.shape, dtype=np.float32)
    s = C.c_void_p()
    assert rt.hipStreamCreate(C.byref(s)) == 0
    g = H.Gpu(plan)
    graph, gexec = C.c_void_p(), C.c_void_p()
    c, h, w = plan.bufs[plan.output]
    din, dout = DevBuf(rt, img.size), DevBuf(rt, c * h * w)
    try:
        ref = g.run(img)
        print("noalloc: S-2 128x128 on the caller's stream", flush=True)
        assert np.array_equal(_pass(rt, g, img, s.value), ref)
        din.put(img)
        print("noalloc: captured into the caller's graph", flush=True)
        assert rt.hipStreamBeginCapture(s, 0) == 0  # hipStreamCaptureModeGlobal
        g.run_noalloc(din.p.value, dout.p.value, s.value)
        assert rt.hipStreamEndCapture(s, C.byref(graph)) == 0
        assert rt.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0) == 0
        for k in range(3):
            dout.put(np.full(c * h * w, np.nan, np.float32))
            assert rt.hipGraphLaunch(gexec, s) == 0
            assert rt.hipStreamSynchronize(s) == 0
            assert np.array_equal(dout.get().reshape(c, h, w), ref), "replay %d" % k
            assert np.array_equal(g.run(img), ref)  # the executor's own eager pass in between
    finally:
        if gexec.value:
            rt.hipGraphExecDestroy(gexec)
        if graph.value:
            rt.hipGraphDestroy(graph)
        din.free()
        dout.free()
        g.close()
        rt.hipStreamDestroy(s)
