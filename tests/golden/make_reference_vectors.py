"""Writes tests/golden/reference_*.npz: golden vectors that pin the MAXIM graph
wiring (the op order and connectivity of the reference builder,
src/model.rs:400-1076), which no published count or size pins.

They come from the reference's own PyTorch transcription of the model,
tools/reference.py (`Maxim`, tools/reference.py:223-583), run in the build
container only, on this repo's seeded random-init checkpoint (Flax names and
layouts) at the smallest input each variant accepts. Nothing here runs on the
GPU box and the reference does not travel: only the vectors are committed.

Each file holds the input image, a SHA-256 of the checkpoint the vectors were
made with (so a change to the weight generator is detected instead of read as
a wiring bug), and a handful of named activations of the reference's trace.

    python tests/golden/make_reference_vectors.py /root/reference
"""

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "maxim-rs_amd"))

# The vectors: (variant, side, seed, gain) and the named activations kept.
CASES = [
    ("S-2", 64, 1, 0.3, ["final", "stage0_out0", "stage0_out1", "stage0_out2", "stage0_global",
                         "stage1_global", "stage0_skip2", "stage1_out2"]),
    ("S-3", 64, 1, 0.3, ["final", "stage0_out0", "stage1_out0", "stage2_global"]),
]


def checkpoint_digest(flat):
    h = hashlib.sha256()
    for k in sorted(flat):
        h.update(k.encode())
        h.update(np.ascontiguousarray(flat[k], np.float32).tobytes())
    return h.hexdigest()


def synthetic(variant, seed, gain):
    from maxim_amd import plan as P
    return P.Weights.synthetic(variant, seed=seed, gain=gain, bias_std=0.02, ln_std=0.1)


def image(side, seed):
    return np.random.default_rng(100 + seed).random((3, side, side), dtype=np.float32)


def main(reference_root):
    import torch
    sys.path.insert(0, os.path.join(reference_root, "tools"))
    import reference  # the reference's own transcription, tools/reference.py

    torch.set_num_threads(8)
    for variant, side, seed, gain, keep in CASES:
        w = synthetic(variant, seed, gain)
        flat = w.flat()
        img = image(side, seed)
        m = reference.Maxim(flat, reference.model_config(variant))
        m.trace = {}
        with torch.no_grad():
            outs = m(torch.from_numpy(img)[None])
        trace = dict(m.trace)
        trace["final"] = outs[-1][-1]
        arrays = {"input": img, "digest": np.frombuffer(checkpoint_digest(flat).encode(), np.uint8)}
        for k in keep:
            arrays[k] = trace[k][0].numpy().astype(np.float32)
        path = os.path.join(HERE, "reference_%s_%d.npz" % (variant.replace("-", ""), side))
        np.savez_compressed(path, **arrays)
        print("wrote %s (%s)" % (path, ", ".join(keep)))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
