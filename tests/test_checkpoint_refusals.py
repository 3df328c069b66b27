"""The safetensors reader (src/weights.rs:37-41's role; the checkpoint is
the command line's other untrusted input) against malformed files: each is
refused with the library's error and nothing it could not hold is
allocated - short files, header lengths past the file, headers that are not
JSON objects or nest without end, shapes that are negative, fractional or
overflow, offsets past the file or reversed, byte counts that do not match,
unknown dtypes, tensors that are not a MAXIM checkpoint - and a real
checkpoint truncated, or with header bytes changed at random, either still
loads or is refused. Also run against the sanitized library (make
sanitize)."""

import json
import struct

import numpy as np
import pytest

from conftest import weights


def P():
    from maxim_amd import plan
    return plan


def st_file(path, header, data=b"", hlen=None):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    open(path, "wb").write(struct.pack("<Q", len(h) if hlen is None else hlen) + h + data)
    return path


def refused(path, match=None):
    with pytest.raises(P().MaximError, match=match):
        P().Weights.open(str(path))


def t(dtype, shape, a, b):
    return {"dtype": dtype, "shape": shape, "data_offsets": [a, b]}


@pytest.mark.parametrize("name,header,data,match", [
    ("short", None, None, "not a safetensors file"),
    ("not_object", [1, 2, 3], b"", "not an object"),
    ("bad_json", b'{"a": {"dtype": "F32", ', b"", "safetensors header"),
    ("deep", b"[" * 100000 + b"]" * 100000, b"", "nested too deeply"),
    ("negative_shape", {"x": t("F32", [-4, 2], 0, 8)}, b"\0" * 8, "bad shape"),
    ("fractional_shape", {"x": t("F32", [1.5, 2], 0, 12)}, b"\0" * 12, "bad shape"),
    ("huge_shape", {"x": t("F32", [1 << 40, 1 << 10], 0, 16)}, b"\0" * 16, "wrong byte count"),
    ("overflow_shape", {"x": t("F32", [1 << 32, 1 << 32, 16], 0, 0)}, b"", "too large"),
    ("wrapping_count", {"x": t("F32", [1 << 30, 1 << 32], 0, 0)}, b"", "wrong byte count"),
    ("beyond_double", {"x": t("F32", [1 << 62], 0, 0)}, b"", "bad shape"),
    ("past_file", {"x": t("F32", [4], 0, 16)}, b"\0" * 8, "runs past the file"),
    ("reversed", {"x": t("F32", [0], 8, 0)}, b"\0" * 8, "runs past the file"),
    ("text_offset", {"x": {"dtype": "F32", "shape": [1], "data_offsets": ["0", "4"]}}, b"\0" * 4, "bad data offset"),
    ("count_mismatch", {"x": t("F32", [3], 0, 8)}, b"\0" * 8, "wrong byte count"),
    ("f16_count", {"x": t("F16", [3], 0, 8)}, b"\0" * 8, "wrong byte count"),
    ("dtype", {"x": t("I8", [8], 0, 8)}, b"\0" * 8, "unsupported dtype"),
    ("incomplete", {"x": {"dtype": "F32", "shape": [2]}}, b"\0" * 8, "incomplete entry"),
    ("not_maxim", {"x": t("F32", [2], 0, 8)}, b"\0" * 8, "not a converted MAXIM checkpoint"),
])
def test_malformed_checkpoint_is_refused(tmp_path, name, header, data, match):
    path = str(tmp_path / (name + ".safetensors"))
    if header is None:
        open(path, "wb").write(b"\x10\x00\x00")
    else:
        st_file(path, header, data)
    refused(path, match)


def test_header_length_past_the_file(tmp_path):
    refused(st_file(str(tmp_path / "a.safetensors"), {"x": t("F32", [1], 0, 4)}, b"\0" * 4, hlen=1 << 20),
            "truncated header")
    refused(st_file(str(tmp_path / "b.safetensors"), b"{}", b"", hlen=(1 << 30) + 1), "not a safetensors file")


def test_real_checkpoint_truncated_or_corrupted(tmp_path):
    ckpt = str(tmp_path / "s2.safetensors")
    weights("S-2").save(ckpt)
    good = open(ckpt, "rb").read()
    assert P().Weights.open(ckpt).count > 100
    hlen = struct.unpack("<Q", good[:8])[0]
    bad = str(tmp_path / "bad.safetensors")
    for n in sorted({0, 7, 8, 9, 100, hlen // 2, hlen + 7, hlen + 8, hlen + 9, len(good) // 2, len(good) - 1}):
        open(bad, "wb").write(good[:n])
        refused(bad)
    rng = np.random.default_rng(3)
    loaded = 0
    for trial in range(150):
        d = bytearray(good[:8 + hlen])
        for _ in range(int(rng.integers(1, 4))):
            d[int(rng.integers(8, 8 + hlen))] = int(rng.choice(list(b'{}[]",:0123456789-.eE ')))
        open(bad, "wb").write(bytes(d) + good[8 + hlen:])
        try:
            P().Weights.open(bad)
            loaded += 1
        except P().MaximError:
            pass
    print("%d of 150 corrupted headers still loaded" % loaded)
