"""Validation-time image handling (CPU): NImage.createImage's load at the
file's own size with a requested channel count (stb_image's conversion),
NImage.resizeMin's integer sizes, NImage.crop's clamped window, and their
composition for one validation image (Classifier.validateSingle,
Classifier.c:420-427)."""
import numpy as np
import pytest

import aetcnn
from test_augment import planes, png_bytes


def rgb_to_grey(pix):
    p = pix.astype(np.int64)
    return ((p[..., 0] * 77 + p[..., 1] * 150 + p[..., 2] * 29) >> 8).astype(np.uint8)


@pytest.mark.parametrize("ctype,bpp", [(0, 1), (2, 3), (4, 2), (6, 4)])
@pytest.mark.parametrize("c", [1, 3, 4])
def test_image_read_converts_channels(tmp_path, ctype, bpp, c):
    rng = np.random.default_rng(10 * ctype + c)
    pix = rng.integers(0, 256, (11, 13, bpp), dtype=np.uint8)
    p = tmp_path / "a.png"
    p.write_bytes(png_bytes(pix, ctype, [0, 4]))
    grey = pix[..., 0] if bpp <= 2 else rgb_to_grey(pix)
    rgb = np.repeat(pix[..., :1], 3, axis=2) if bpp <= 2 else pix[..., :3]
    alpha = pix[..., -1] if bpp in (2, 4) else np.full(pix.shape[:2], 255, np.uint8)
    want = {1: grey[..., None], 3: rgb, 4: np.concatenate([rgb, alpha[..., None]], axis=2)}[c]
    got = aetcnn.image_read(str(p), c)
    assert got.shape == (c, 11, 13)
    assert np.array_equal(got, planes(want))


def test_image_read_ppm_any_size(tmp_path):
    rng = np.random.default_rng(4)
    pix = rng.integers(0, 256, (5, 17, 3), dtype=np.uint8)
    p = tmp_path / "a.ppm"
    p.write_bytes(b"P6\n17 5\n255\n" + pix.tobytes())
    assert np.array_equal(aetcnn.image_read(str(p), 3), planes(pix))


def test_resize_min_sizes():
    # the smaller side becomes min, the other scales in integer arithmetic
    assert aetcnn.resize_min_size(40, 36, 32) == (35, 32)
    assert aetcnn.resize_min_size(20, 50, 32) == (32, 80)
    assert aetcnn.resize_min_size(64, 64, 32) == (32, 32)
    assert aetcnn.resize_min_size(32, 32, 32) == (32, 32)
    assert aetcnn.resize_min_size(33, 100, 32) == (32, 96)


def test_crop_window_and_clamp():
    src = np.arange(2 * 4 * 5, dtype=np.float32).reshape(2, 4, 5)
    assert np.array_equal(aetcnn.image_crop(src, 1, 2, 3, 2), src[:, 2:4, 1:4])
    # coordinates outside the image take the nearest edge pixel
    got = aetcnn.image_crop(src, -2, 3, 3, 2)
    rows = np.clip(np.arange(3, 5), 0, 3)
    cols = np.clip(np.arange(-2, 1), 0, 4)
    assert np.array_equal(got, src[:, rows][:, :, cols])


def test_validation_image_composition(tmp_path):
    rng = np.random.default_rng(7)
    # exactly the input size: no resize, no crop
    pix = rng.integers(0, 256, (32, 32, 3), dtype=np.uint8)
    p = tmp_path / "same.png"
    p.write_bytes(png_bytes(pix, 2, [1]))
    assert np.array_equal(aetcnn.validation_image(str(p), 32, 32, 3), planes(pix))
    # twice the size: the bilinear resize only (already pinned in test_augment)
    pix = rng.integers(0, 256, (64, 64, 3), dtype=np.uint8)
    p = tmp_path / "big.png"
    p.write_bytes(png_bytes(pix, 2, [2]))
    assert np.array_equal(aetcnn.validation_image(str(p), 32, 32, 3),
                          aetcnn.image_resize(planes(pix), 32, 32))
    # wide grey image: resized to 51 x 32, then the centre 32 columns from 9
    pix = rng.integers(0, 256, (40, 64, 1), dtype=np.uint8)
    p = tmp_path / "wide.png"
    p.write_bytes(png_bytes(pix, 0, [3]))
    rs = aetcnn.image_resize(planes(np.repeat(pix, 3, axis=2)), 51, 32)
    assert np.array_equal(aetcnn.validation_image(str(p), 32, 32, 3), rs[:, :, 9:41])
