"""The drop-in boundary: the product library loads, exports every entry point
the headers declare, and reports errors the way the reference's
`maxim::Error` does (a message, never a crash). No device work here."""

import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "maxim-rs_amd", "lib", "libmaxim_hip.so")


def declared():
    names = []
    for h in ("maxim_plan.h", "maxim_hip.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(mxh?_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) >= 45, names
    lib = C.CDLL(LIB)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_no_link_time_hip_dependency():
    """The HIP runtime is dlopen'd (as the reference dlopens libcuda), so the
    library's dynamic section names no ROCm library."""
    import subprocess
    out = subprocess.run(["readelf", "-d", LIB], capture_output=True, text=True).stdout
    needed = re.findall(r"Shared library: \[(.*?)\]", out)
    assert needed and not any("amdhip" in n or "hsa" in n or "roc" in n for n in needed), needed


def test_the_code_object_is_embedded_and_complete():
    """Every kernel the executor can launch is in the embedded gfx950 code
    object (the reference checks its kernel list both ways at startup,
    src/cuda.rs:76-85)."""
    data = open(LIB, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    src = open(os.path.join(ROOT, "maxim-rs_amd", "csrc", "exec", "exec_hip.cpp")).read()
    launched = set(re.findall(r'"(mx_[a-z0-9_]+)"', src))
    launched |= {"mx_gemm_%dx%d%s" % (m, n, v) for m, n in ((128, 128), (64, 128), (128, 64), (64, 64),
                                                           (32, 128), (32, 64))
                 for v in ("", "_v4", "_f", "_v4_f", "_t", "_v4_t")}
    launched |= {"mx_conv3x3_m%d_t%d%s%s" % (m, t, s, f) for m in (32, 64, 128) for t in (4, 8)
                 for s in ("", "_c4") for f in ("", "_f")}
    launched |= {"mx_conv4x4_m%d_t%d%s" % (m, t, z) for m in (32, 64, 128) for t in (4, 8) for z in ("", "_s")}
    launched |= {"mx_conv3x3%s_m16_t8%s" % (v, f) for v in ("", "v") for f in ("", "_f")}
    launched |= {"mx_wino3_t%d%s" % (t, f) for t in (4, 8, 16) for f in ("", "_f", "_f_e16")}
    launched |= {"mx_conv3x3v_m%d_t%d%s" % (m, t, f) for m in (32, 64, 128) for t in (4, 8) for f in ("", "_f")}
    launched |= {"mx_pw_%s%d%s%s" % (l, t, k, f) for l in ("ch", "rw") for t in (1, 2, 4)
                 for k in ("", "_k4") for f in ("", "_f")}
    launched |= {"mx_pw_ch%d%s_ln%s" % (t, k, f) for t in (1, 2, 4) for k in ("", "_k4") for f in ("", "_f")}
    launched |= {"mx_pw_%s%d%s_xm%s" % (l, t, k, f) for l in ("ch", "rw") for t in (1, 2, 4)
                 for k in ("", "_k4") for f in ("", "_f")}
    # the channel-major forms over a folded batch (GateMm mode 0)
    launched |= {"mx_pw_chb%d%s%s%s" % (t, k, x, f) for t in (1, 2, 4) for k in ("", "_k4") for x in ("", "_xm")
                 for f in ("", "_f")}
    launched |= {"mx_pw_chb2_k4_f_e65"}
    launched |= {"mx_pw_ch%d%s_mul%s" % (t, k, f) for t in (1, 2, 4) for k in ("", "_k4") for f in ("", "_f")}
    launched |= {"mx_pw_ch%d%s_t" % (t, k) for t in (1, 2, 4) for k in ("", "_k4")}
    launched |= {"mx_pw_ch%d%s%s_f_lo" % (t, k, l) for t in (2, 4) for k in ("", "_k4") for l in ("", "_ln")}
    launched |= {"mx_pw_ch1_f_lo", "mx_pw_ch1_f_lo_e66"}
    launched |= {"mx_c3_m%d_t%d%s" % (m, t, f) for m, t in ((32, 8), (64, 4), (64, 2)) for f in ("", "_f")}
    launched |= {"mx_resize_hv%s_t%d" % (v, t) for v in ("", "4") for t in (2, 4, 8)}
    launched |= {"mx_chan%s_c%d%s" % (s, c, p) for s in ("_ln", "_ln_stats", "_scale_add_stats")
                 for c in (32, 64, 128) for p in ("", "_p%d" % (4096 // c), "_p%d" % (2048 // c))}
    # the paired forms of the streaming kernels a multi-axis gMLP block's
    # branches share (the executor appends _x2 to the step's kernel)
    launched |= {"mx_pw_ch2_ln_f_lo_e72_x2", "mx_pw_ch1_f_e226_x2", "mx_pw_ch2_f_e226_x2", "mx_pw_ch2_k4_f_e226_x2"}
    launched = {k for k in launched if not k.endswith("_") and not k.endswith("_c")}
    missing = [k for k in sorted(launched) if k.encode() + b"\0" not in data]
    assert not missing, missing


def test_errors_are_messages():
    from maxim_amd import plan as P
    from maxim_amd import hip as H
    with pytest.raises(P.MaximError, match="cannot open"):
        P.Weights.open("/nonexistent.safetensors")
    assert "cannot open" in P.last_error()
    # An op whose dimensions disagree with its buffers is refused before any
    # device work (the executor validates the whole plan first).
    op = P.make_op(P.CONV3X3, dst=1, src=0, w=0, c_in=4, c_out=8, h=5, wd=5)
    cp = P.CustomPlan([(4, 5, 5), (8, 5, 6)], [op], [[0.0] * (9 * 4 * 8)])
    with pytest.raises(P.MaximError, match="conv3x3 out"):
        H.Gpu(cp)
    op = P.make_op(P.ADD, dst=2, src=0, src2=7, n=4)
    cp = P.CustomPlan([(1, 2, 2)] * 3, [op], [])
    with pytest.raises(P.MaximError, match="buffer 7"):
        H.Gpu(cp)
