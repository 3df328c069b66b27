"""The plan contract: known-answer tests from the reference's published
numbers, and the reference's own plan-level property tests
(tests/arena.rs, tests/packing.rs) with seeded weights instead of the LOL
checkpoint. No op is executed here except the graph-wiring golden check.
"""

import hashlib
import importlib.util
import os

import numpy as np
import pytest

from conftest import buf, run_oracle, weights

HERE = os.path.dirname(os.path.abspath(__file__))


def P():
    from maxim_amd import plan
    return plan


# (variant, h, w, ops, buffers, arena MiB, weight MiB) - docs/DEVELOPING.md:100-105,
# 137-144; README.md:107-110. Weight MiB include the GPU build's layout twins.
KATS = [
    ("S-2", 256, 256, 1840, 2089, 115.0, 86.7),
    ("S-3", 256, 256, 2885, 3276, 115.0, 135.2),
    ("S-2", 448, 640, 1840, 2089, 503.1, 86.7),
    ("S-3", 768, 704, 2885, 3276, 948.6, 135.2),
    ("S-2", 2048, 2048, 1840, 2089, 7359.0, 86.7),
    ("S-2", 4096, 4096, 1840, 2089, 29436.0, 86.7),
]


@pytest.mark.parametrize("variant,h,w,ops,bufs,arena,wmib", KATS)
def test_plan_size_kats(variant, h, w, ops, bufs, arena, wmib):
    plan = P().Plan(weights(variant), h, w)
    assert len(plan.ops) == ops
    assert len(plan.bufs) == bufs
    assert round(plan.arena_bytes / 2**20, 1) == arena
    assert round(plan.weight_bytes / 2**20, 1) == wmib


def test_checkpoint_kats():
    # README.md:54-70 (14.2 M / 22.2 M params); src/host.rs:9 (1760 tensors, S-2).
    s2, s3 = weights("S-2"), weights("S-3")
    assert s2.count == 1760
    assert round(s2.params / 1e6, 1) == 14.2 and round(s3.params / 1e6, 1) == 22.2
    assert (s2.config.features, s2.config.num_stages) == (32, 2)
    assert (s3.config.features, s3.config.num_stages) == (32, 3)


def live_set_peak(plan):
    """tests/arena.rs:38-82: the true live-set peak, charged to owning buffers."""
    n = len(plan.bufs)

    def root(i):
        a = plan.alias(i)
        return i if a is None else root(a[0])

    owner = [root(i) for i in range(n)]
    first, last = {}, {}
    for oi, op in enumerate(plan.ops):
        for b in plan.operands(op):
            b = owner[b]
            first.setdefault(b, oi)
            last[b] = oi
    ev = np.zeros(len(plan.ops) + 1, np.int64)
    for b in first:
        ev[first[b]] += plan.buf_len(b) * 4
        ev[last[b] + 1] -= plan.buf_len(b) * 4
    return int(np.cumsum(ev).max())


def test_the_arena_is_close_to_the_live_set():
    """tests/arena.rs:84-106: arena <= 1.20x the live-set peak; the 2048^2 peak
    is the published 6847.0 MiB."""
    for h, w in [(480, 640), (832, 1280)]:
        plan = P().Plan(weights("S-2"), h, w)
        ratio = plan.arena_bytes / live_set_peak(plan)
        assert ratio <= 1.20, (h, w, ratio)
    plan = P().Plan(weights("S-2"), 2048, 2048)
    assert round(live_set_peak(plan) / 2**20, 1) == 6847.0


def test_naming_activations_is_what_costs_the_memory():
    """tests/arena.rs:108-126."""
    named = P().Plan(weights("S-2"), 480, 640, named=True)
    lean = P().Plan(weights("S-2"), 480, 640)
    assert len(named.dumps) == 43
    assert named.arena_bytes / lean.arena_bytes > 1.5


def test_named_buffers_fit_the_arena():
    """tests/packing.rs:69-85."""
    plan = P().Plan(weights("S-2"), 64, 64, named=True)
    for name, b in plan.dumps:
        assert int(plan.offs[b]) + plan.buf_len(b) <= plan.arena_len, name


@pytest.mark.parametrize("variant,h,w", [("S-2", 64, 64), ("S-3", 448, 640)])
def test_no_op_overlaps_its_own_inputs(variant, h, w):
    """tests/packing.rs:87-118."""
    plan = P().Plan(weights(variant), h, w)
    bad = []
    for i, op in enumerate(plan.ops):
        ids = plan.operands(op)
        d, dn = int(plan.offs[ids[0]]), plan.buf_len(ids[0])
        for s in ids[1:]:
            so, sn = int(plan.offs[s]), plan.buf_len(s)
            if d < so + sn and so < d + dn:
                bad.append((i, op.describe()))
    assert not bad, bad[:5]


def test_dumps_do_not_change_the_result():
    """tests/packing.rs:54-67: the same 64x64 graph with and without names is
    bit-identical through the CPU path."""
    w = weights("S-2")
    img = np.random.default_rng(3).random((3, 64, 64), dtype=np.float32)
    outs = []
    for named in (True, False):
        plan = P().Plan(w, 64, 64, named=named)
        outs.append(buf(plan, run_oracle(plan, img), plan.output).copy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_too_small_for_the_model_is_refused():
    with pytest.raises(P().MaximError, match="too small for this model"):
        P().Plan(weights("S-2"), 32, 32)


def test_safetensors_roundtrip(tmp_path):
    """The tools/convert.py layout written and read back: same tensors, the
    variant derived from the file (src/config.rs:71-100), the same plan."""
    path = str(tmp_path / "s3.safetensors")
    w = weights("S-3")
    w.save(path, task="denoising")
    raw = open(path, "rb").read()
    hlen = int.from_bytes(raw[:8], "little")
    assert (8 + hlen) % 8 == 0
    import json
    hdr = json.loads(raw[8:8 + hlen])
    assert hdr["__metadata__"]["format"] == "maxim" and hdr["__metadata__"]["variant"] == "S-3"
    assert hdr["__metadata__"]["tensor_count"] == str(w.count)
    keys = [k for k in hdr if k != "__metadata__"]
    assert keys == sorted(keys)
    r = P().Weights.open(path)
    assert (r.config.features, r.config.num_stages) == (32, 3)
    assert r.count == w.count
    for name in ("stage_0_encoder_block_0/Conv_0/kernel", "UpSampleRatio_3/Conv_0/bias",
                 "stage_2_output_conv_1/kernel"):
        assert np.array_equal(r.tensor(name), w.tensor(name))
    a, b = P().Plan(w, 128, 128), P().Plan(r, 128, 128)
    assert a.arena_len == b.arena_len and np.array_equal(a.offs, b.offs)
    for i in range(a.n_weights):
        assert np.array_equal(a.weight(i), b.weight(i))


def test_checkpoint_errors(tmp_path):
    with pytest.raises(P().MaximError, match="cannot open"):
        P().Weights.open(str(tmp_path / "missing.safetensors"))
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(b"\x10\x00\x00\x00\x00\x00\x00\x00{\"a\":1}        ")
    with pytest.raises(P().MaximError):
        P().Weights.open(str(bad))


def test_variant_table():
    """src/config.rs:33-60 and :101-116."""
    for v, (f, s) in {"S-1": (32, 1), "S-2": (32, 2), "S-3": (32, 3), "M-1": (64, 1),
                      "M-2": (64, 2), "M-3": (64, 3)}.items():
        c = P().config(v)
        assert (c.features, c.num_stages, c.depth, c.num_groups) == (f, s, 3, 2)
        assert (c.block_size_hr, c.block_size_lr, c.grid_size_hr, c.grid_size_lr) == (16, 8, 16, 8)
    with pytest.raises(P().MaximError, match="unknown variant"):
        P().config("L-9")


def test_weight_transforms():
    """src/weights.rs:57-211 as index maps of the Flax tensors: conv1x1 and Dense
    -> [co][ci], kxk -> [co][ci][k][k], 3x3 twin [tap][ci][co], convT ->
    [ci][co][2][2] spatially reversed, gating Dense -> [out][in]."""
    w = weights("S-2")
    plan = P().Plan(w, 64, 64)
    seen = set()
    from maxim_amd import plan as PP
    for op in plan.ops:
        if op.kind == PP.CONV3X3 and "3x3" not in seen:
            k = plan.weight(op.w).reshape(op.c_out, op.c_in, 3, 3)
            t = plan.weight(op.wt).reshape(3, 3, op.c_in, op.c_out)
            assert np.array_equal(k, t.transpose(3, 2, 0, 1))
            seen.add("3x3")
        if op.kind == PP.CONV1X1 and "1x1" not in seen:
            k = plan.weight(op.w).reshape(op.c_out, op.c_in)
            t = plan.weight(op.wt).reshape(op.c_in, op.c_out)
            assert np.array_equal(k, t.T)
            seen.add("1x1")
    k = w.tensor("stage_0_cross_gating_block_0/ConvTranspose_0/kernel")  # [2][2][ci][co], first 64->32
    conv = next(op for op in plan.ops if op.kind == PP.CONVT2X2 and op.c_out == 32 and op.h == 32)
    t = plan.weight(conv.w).reshape(conv.c_in, conv.c_out, 2, 2)
    assert np.array_equal(t, k[::-1, ::-1].transpose(2, 3, 0, 1))
    assert seen == {"3x3", "1x1"}


def _load_maker():
    spec = importlib.util.spec_from_file_location(
        "make_reference_vectors", os.path.join(HERE, "golden", "make_reference_vectors.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


@pytest.mark.parametrize("case", [0, 1])
def test_graph_wiring_matches_the_reference_transcription(case):
    """The graph wiring against golden vectors written by the reference's own
    model transcription (tools/reference.py) on the same seeded checkpoint and
    input. The CPU path differs from it only in the resize implementation and
    the LayerNorm variance formula (both documented there), so agreement is to
    float rounding: max-abs <= 1e-5 * max|ref| on every kept activation."""
    mk = _load_maker()
    variant, side, seed, gain, keep = mk.CASES[case]
    z = np.load(os.path.join(HERE, "golden", "reference_%s_%d.npz" % (variant.replace("-", ""), side)))
    w = mk.synthetic(variant, seed, gain)
    assert bytes(z["digest"]).decode() == mk.checkpoint_digest(w.flat()), \
        "the seeded checkpoint changed: regenerate tests/golden with make_reference_vectors.py"
    plan = P().Plan(w, side, side, named=True)
    arena = run_oracle(plan, z["input"])
    names = dict(plan.dumps)
    for k in keep:
        ref = z[k]
        got = buf(plan, arena, names[k]).reshape(ref.shape)
        err = float(np.abs(got.astype(np.float64) - ref).max())
        assert err <= 1e-5 * float(np.abs(ref).max()), (k, err)


def test_input_sides_beyond_the_limit_are_refused():
    """A side over 2^24 pixels is refused by name (past it, buffer sizes and
    arena offsets would overflow 64 bits and wrap to a small arena); at the
    limit every size is still exact: the arena holds the largest buffer."""
    from maxim_amd import plan as P
    w = weights("S-2")
    for h, wd in [(64, (1 << 24) + 64), ((1 << 40), (1 << 40)), ((1 << 62), (1 << 62))]:
        with pytest.raises(P.MaximError, match="limited to 16777216"):
            P.Plan(w, h, wd)
    p = P.Plan(P.Weights.synthetic("M-3", seed=1), 1 << 24, 1 << 24)
    largest = max(c * h * ww for c, h, ww in p.bufs)
    assert largest >= 64 * (1 << 48)  # the full-resolution features, 64 channels of 2^48 pixels
    assert p.arena_len >= largest and p.arena_len * 4 < (1 << 64)
