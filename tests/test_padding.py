"""The reference pipeline's padding (src/image.rs:106-246), with the known
answers of the reference's tests/padding.rs, plus numpy's reflect pad as the
library check of the padded values and the crop as its exact inverse."""

import numpy as np
import pytest


def P():
    from maxim_amd import plan
    return plan


def rgb(h, w):
    return ((np.arange(3 * h * w) % 251) / 251.0).astype(np.float32).reshape(3, h, w)


def test_a_sixteen_pixel_image_is_refused_with_the_numbers():
    with pytest.raises(P().MaximError) as e:
        P().preprocess(rgb(16, 16), 64)
    m = str(e.value)
    assert "too small" in m
    assert "height is 16 pixels" in m
    assert "24 pixels of padding a side" in m
    assert "at least 22 pixels" in m


def test_one_axis_over_the_line_is_refused_by_name():
    with pytest.raises(P().MaximError) as e:
        P().preprocess(rgb(64, 16), 64)
    m = str(e.value)
    assert "width is 16 pixels" in m and "the height is 16" not in m


def test_a_square_over_the_boundary_pads_to_one_factor_block():
    p = P().preprocess(rgb(32, 32), 64)
    assert p.img.shape[1:] == (64, 64)
    assert (p.even_h, p.even_w, p.orig_h, p.orig_w) == (32, 32, 32, 32)


def test_the_boundary_itself_is_accepted():
    assert P().preprocess(rgb(22, 22), 64).img.shape[1:] == (64, 64)


def test_an_odd_size_is_made_even_first_and_still_pads():
    p = P().preprocess(rgb(33, 33), 64)
    assert (p.even_h, p.even_w) == (34, 34)
    assert p.img.shape == (3, 64, 64)


@pytest.mark.parametrize("h,w", [(400, 600), (33, 47), (64, 128), (669, 760)])
def test_values_are_numpy_reflect_and_crop_inverts(h, w):
    img = np.random.default_rng(h * w).random((3, h, w), dtype=np.float32)
    p = P().preprocess(img, 64)
    even = np.pad(img, ((0, 0), (0, h % 2), (0, w % 2)), mode="reflect")
    ph, pw = p.img.shape[1] - even.shape[1], p.img.shape[2] - even.shape[2]
    want = np.pad(even, ((0, 0), (ph // 2, ph // 2), (pw // 2, pw // 2)), mode="reflect")
    assert np.array_equal(p.img, want)
    assert p.img.shape[1] % 64 == 0 and p.img.shape[2] % 64 == 0
    assert np.array_equal(P().crop_out(p.img, p), img)


def test_c4_geometry():
    """600x400 pads to 640x448: 24 rows top and bottom, 20 columns left and right."""
    img = np.random.default_rng(0).random((3, 400, 600), dtype=np.float32)
    p = P().preprocess(img, 64)
    assert p.img.shape == (3, 448, 640)
    assert np.array_equal(p.img[:, 24:424, 20:620], img)


def test_same_pad():
    """flax SAME (src/image.rs:106-111): ceil(size/stride) outputs, larger pad last."""
    for size in range(1, 40):
        for stride, k in [(2, 4), (1, 3), (2, 3)]:
            a, b = P().same_pad(size, stride, k)
            out = -(-size // stride)
            assert a + b == max((out - 1) * stride + k - size, 0) and b - a in (0, 1)
    assert P().same_pad(448, 2, 4) == (1, 1)
