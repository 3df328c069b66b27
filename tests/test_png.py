"""PNG in and out (the reference's image::read_png / write_png,
src/image.rs:33-104, over the `png` crate): the library's decoder against
files written here with Python's zlib at every compression level (stored,
fixed- and dynamic-Huffman deflate blocks) and every row filter, in every
8-bit colour type the reference accepts; its encoder against a decoder
written here; the reference's rounding (half up after clamping) and its
refusal of indexed images."""

import struct
import zlib

import numpy as np
import pytest

from conftest import ROOT  # noqa: F401  (sets sys.path)


def P():
    from maxim_amd import plan
    return plan


def chunk(t, data):
    return struct.pack(">I", len(data)) + t + data + struct.pack(">I", zlib.crc32(t + data) & 0xffffffff)


def paeth(a, b, c):
    p = a + b - c
    pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
    return a if pa <= pb and pa <= pc else (b if pb <= pc else c)


def filter_rows(px, ch, filters):
    """Filter each row of px ([h][w*ch] uint8) with the given filter types."""
    h, stride = px.shape
    raw = bytearray()
    for y in range(h):
        ft = filters[y % len(filters)]
        raw.append(ft)
        for x in range(stride):
            a = int(px[y, x - ch]) if x >= ch else 0
            b = int(px[y - 1, x]) if y else 0
            c = int(px[y - 1, x - ch]) if (y and x >= ch) else 0
            pred = [0, a, b, (a + b) >> 1, paeth(a, b, c)][ft]
            raw.append((int(px[y, x]) - pred) & 0xff)
    return bytes(raw)


def write_test_png(path, px, ctype, level, filters=(0, 1, 2, 3, 4), depth=8, interlace=0):
    h, w, ch = px.shape
    raw = filter_rows(px.reshape(h, w * ch), ch, filters)
    data = b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, depth, ctype, 0, 0, interlace))
    z = zlib.compress(raw, level)
    # split the stream over two IDAT chunks, as encoders may
    data += chunk(b"IDAT", z[: len(z) // 2]) + chunk(b"IDAT", z[len(z) // 2:]) + chunk(b"IEND", b"")
    open(path, "wb").write(data)


def decode_test_png(path):
    """A plain decoder for the library's own output: 8-bit RGB."""
    d = open(path, "rb").read()
    assert d[:8] == b"\x89PNG\r\n\x1a\n"
    at, z, ihdr = 8, b"", None
    while at < len(d):
        n = struct.unpack(">I", d[at:at + 4])[0]
        t, body = d[at + 4:at + 8], d[at + 8:at + 8 + n]
        assert struct.unpack(">I", d[at + 8 + n:at + 12 + n])[0] == zlib.crc32(t + body) & 0xffffffff
        if t == b"IHDR":
            ihdr = struct.unpack(">IIBBBBB", body)
        elif t == b"IDAT":
            z += body
        at += 12 + n
    w, h, depth, ctype = ihdr[:4]
    assert depth == 8 and ctype == 2
    raw = zlib.decompress(z)
    rows = []
    prev = bytearray(w * 3)
    for y in range(h):
        ft = raw[y * (w * 3 + 1)]
        assert ft == 0
        row = bytearray(raw[y * (w * 3 + 1) + 1:(y + 1) * (w * 3 + 1)])
        rows.append(row)
        prev = row
    return np.frombuffer(b"".join(rows), np.uint8).reshape(h, w, 3)


@pytest.mark.parametrize("ctype,ch", [(2, 3), (6, 4), (0, 1), (4, 2)])
@pytest.mark.parametrize("level", [0, 1, 9])
def test_read_every_colour_type_filter_and_block_kind(tmp_path, ctype, ch, level):
    rng = np.random.default_rng(ctype * 10 + level)
    h, w = 37, 53
    # smooth content (long matches for the compressor) plus noise
    yy, xx = np.mgrid[0:h, 0:w]
    px = ((np.sin(xx / 7.0 + yy / 11.0)[..., None] * 100 + 128 + rng.integers(0, 20, (h, w, ch)))
          .clip(0, 255).astype(np.uint8))
    path = str(tmp_path / "t.png")
    write_test_png(path, px, ctype, level)
    got = P().read_png(path)
    rgb = px[..., :3] if ch >= 3 else np.repeat(px[..., :1], 3, axis=2)
    want = rgb.transpose(2, 0, 1).astype(np.float32) / np.float32(255.0)
    assert got.shape == (3, h, w)
    assert np.array_equal(got, want)


def test_write_rounds_half_up_and_clamps(tmp_path):
    img = np.zeros((3, 4, 5), np.float32)
    img[0, 0, :] = [0.5, -0.25, 1.5, np.nan, 1.0]
    img[1, 1, :] = (np.arange(5) + 0.49) / 255.0
    img[2, 2, :] = np.linspace(0, 1, 5)
    path = str(tmp_path / "o.png")
    P().write_png(path, img)
    got = decode_test_png(path).transpose(2, 0, 1)
    v = np.where(np.isnan(img), 0, np.clip(img, 0, 1))
    want = (v * np.float32(255.0) + np.float32(0.5)).astype(np.uint8)
    assert np.array_equal(got, want)
    assert got[0, 0, 0] == 128 and got[0, 0, 1] == 0 and got[0, 0, 2] == 255 and got[0, 0, 3] == 0
    # the file ends with the IEND chunk, whose CRC is the well-known AE 42 60 82
    assert open(path, "rb").read()[-12:] == b"\x00\x00\x00\x00IEND\xaeB`\x82"


def test_round_trip_large(tmp_path):
    """A 600x400 image (more than one stored deflate block) survives a round
    trip exactly at 8 bits."""
    rng = np.random.default_rng(3)
    q = rng.integers(0, 256, (3, 400, 600)).astype(np.float32) / np.float32(255.0)
    path = str(tmp_path / "r.png")
    P().write_png(path, q)
    assert np.array_equal(P().read_png(path), q)


def test_refusals(tmp_path):
    px = np.zeros((4, 4, 1), np.uint8)
    path = str(tmp_path / "i.png")
    write_test_png(path, px, 3, 9)
    with pytest.raises(P().MaximError, match="indexed PNG; re-save it as RGB"):
        P().read_png(path)
    write_test_png(path, np.zeros((4, 4, 3), np.uint8), 2, 9, depth=16)
    with pytest.raises(P().MaximError, match="16-bit"):
        P().read_png(path)
    d = bytearray(open(path, "rb").read())
    d[20] ^= 1  # a byte inside IHDR: its CRC no longer matches
    open(path, "wb").write(bytes(d))
    with pytest.raises(P().MaximError, match="CRC"):
        P().read_png(path)
    with pytest.raises(P().MaximError):
        P().read_png(str(tmp_path / "missing.png"))


# Adam7 (PNG 1.2, 8.2): pass p takes rows R0[p] + k * DR[p] and columns
# C0[p] + k * DC[p]; each non-empty pass is filtered as an image of its own.
R0, C0 = (0, 0, 4, 0, 2, 0, 1), (0, 4, 0, 2, 0, 1, 0)
DR, DC = (8, 8, 8, 4, 4, 2, 2), (8, 8, 4, 4, 2, 2, 1)


def write_interlaced_png(path, px, ctype, level, filters=(0, 1, 2, 3, 4)):
    h, w, ch = px.shape
    raw = b""
    for p in range(7):
        sub = px[R0[p]::DR[p], C0[p]::DC[p]]
        if sub.shape[0] == 0 or sub.shape[1] == 0:
            continue  # an empty pass contributes no bytes at all
        sh, sw = sub.shape[:2]
        # rotate the filter list per pass so every filter meets every pass
        raw += filter_rows(np.ascontiguousarray(sub).reshape(sh, sw * ch), ch, filters[p % 5:] + filters[:p % 5])
    data = b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, 8, ctype, 0, 0, 1))
    data += chunk(b"IDAT", zlib.compress(raw, level)) + chunk(b"IEND", b"")
    open(path, "wb").write(data)


@pytest.mark.parametrize("h,w", [(37, 53), (1, 1), (1, 9), (5, 1), (3, 3), (8, 8), (17, 16)])
@pytest.mark.parametrize("ctype,ch", [(2, 3), (6, 4), (0, 1), (4, 2)])
def test_read_interlaced(tmp_path, h, w, ctype, ch):
    """Adam7 files (the reference's png crate deinterlaces them in
    next_frame), including sizes where some of the seven passes are empty."""
    rng = np.random.default_rng(h * 100 + w + ctype)
    px = rng.integers(0, 256, (h, w, ch)).astype(np.uint8)
    path = str(tmp_path / "a7.png")
    write_interlaced_png(path, px, ctype, 6)
    got = P().read_png(path)
    rgb = px[..., :3] if ch >= 3 else np.repeat(px[..., :1], 3, axis=2)
    assert np.array_equal(got, rgb.transpose(2, 0, 1).astype(np.float32) / np.float32(255.0))
    # an independent decoder agrees on the file (Pillow deinterlaces on load)
    from PIL import Image
    ref = np.asarray(Image.open(path).convert("RGB"))
    assert np.array_equal(got, ref.transpose(2, 0, 1).astype(np.float32) / np.float32(255.0))


def test_file_from_pillow(tmp_path):
    """A file Pillow's encoder writes (interlacing is not among its save
    options, so this pins the plain path against a third-party encoder)."""
    from PIL import Image
    rng = np.random.default_rng(11)
    px = rng.integers(0, 256, (29, 31, 3)).astype(np.uint8)
    path = str(tmp_path / "pil.png")
    Image.fromarray(px).save(path, optimize=True)
    assert np.array_equal(P().read_png(path), px.transpose(2, 0, 1).astype(np.float32) / np.float32(255.0))


def test_stream_forms(tmp_path):
    """read_png_stream / write_png_stream (the CLI's `-i -` and `-o -`): the
    same image from bytes as from the file, and the encoder's bytes are the
    file's bytes."""
    rng = np.random.default_rng(5)
    q = rng.integers(0, 256, (3, 21, 34)).astype(np.float32) / np.float32(255.0)
    path = str(tmp_path / "s.png")
    P().write_png(path, q)
    data = open(path, "rb").read()
    assert P().encode_png(q) == data
    assert np.array_equal(P().read_png(data=data), q)
    with pytest.raises(P().MaximError, match="not a PNG"):
        P().read_png(data=b"not a png at all")


def test_pixels_refuses_a_short_buffer(tmp_path):
    """The decoded image is copied out only into a buffer that holds it."""
    import ctypes as C
    q = np.zeros((3, 6, 7), np.float32)
    path = str(tmp_path / "c.png")
    P().write_png(path, q)
    lib = P().lib()
    h, w, img = C.c_int64(), C.c_int64(), C.c_void_p()
    assert lib.mx_png_open(path.encode(), None, 0, C.byref(img), C.byref(h), C.byref(w)) == 0
    try:
        out = np.zeros(3 * 6 * 7, np.float32)
        assert lib.mx_png_pixels(img, out.ctypes.data, out.size - 1) != 0
        assert b"needs 126" in lib.mx_last_error()
        assert lib.mx_png_pixels(img, out.ctypes.data, out.size) == 0
    finally:
        lib.mx_png_close(img)


def chunks_of(d):
    """[(type, body)] of a PNG byte string."""
    at, out = 8, []
    while at + 12 <= len(d):
        n = struct.unpack(">I", d[at:at + 4])[0]
        out.append((d[at + 4:at + 8], d[at + 8:at + 8 + n]))
        at += 12 + n
    return out


def assemble(chs):
    return b"\x89PNG\r\n\x1a\n" + b"".join(chunk(t, b) for t, b in chs)


def decodes_or_refuses(data, shape=None):
    """The library either decodes `data` (to the declared shape, values in
    0..1) or refuses it with its own error; anything else fails the test."""
    try:
        img = P().read_png(data=data)
    except P().MaximError:
        return False
    assert img.dtype == np.float32 and img.ndim == 3 and img.shape[0] == 3
    if shape is not None:
        assert img.shape == shape
    assert np.isfinite(img).all() and img.min() >= 0.0 and img.max() <= 1.0
    return True


@pytest.mark.parametrize("interlaced", [False, True])
def test_malformed_inputs_are_refused_not_crashed(tmp_path, interlaced):
    """The decoder reads untrusted files (the command line's input): every
    truncation of a valid file, and bytes of its compressed stream changed
    at random with the CRCs recomputed (so the inflater itself meets them:
    bad block types, Huffman tables, distances past the output, lengths past
    the image), and forged IHDR sizes each either decode to the size the
    header declares or raise the library's error - no crash, no read or
    write outside a buffer (this suite also runs under AddressSanitizer)."""
    rng = np.random.default_rng(7 if interlaced else 8)
    px = rng.integers(0, 256, size=(13, 21, 3), dtype=np.uint8)
    path = str(tmp_path / "ok.png")
    if interlaced:
        write_interlaced_png(path, px, 2, 6)
    else:
        write_test_png(path, px, 2, 6)
    good = open(path, "rb").read()
    assert decodes_or_refuses(good, (3, 13, 21))
    for n in range(len(good)):
        decodes_or_refuses(good[:n], (3, 13, 21))
    chs = chunks_of(good)
    z = b"".join(b for t, b in chs if t == b"IDAT")
    head = [c for c in chs if c[0] == b"IHDR"]
    decoded = 0
    for trial in range(400):
        zz = bytearray(z)
        for _ in range(int(rng.integers(1, 4))):
            at = int(rng.integers(2, len(zz)))  # keep the zlib header, so inflate is reached
            zz[at] = int(rng.integers(0, 256))
        decoded += decodes_or_refuses(assemble(head + [(b"IDAT", bytes(zz)), (b"IEND", b"")]), (3, 13, 21))
    print("%d of 400 corrupted streams still decoded" % decoded)
    w_h = [(0, 5), (5, 0), (1 << 20, 1), (1, (1 << 20) + 1), (0xffffffff, 0xffffffff), (30000, 30000), (22, 13)]
    for w, h in w_h:
        ihdr = struct.pack(">IIBBBBB", w, h, 8, 2, 0, 0, 1 if interlaced else 0)
        data = assemble([(b"IHDR", ihdr), (b"IDAT", z), (b"IEND", b"")])
        assert not decodes_or_refuses(data), (w, h)
