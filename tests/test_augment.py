"""The input pipeline's image decoding and augmentation on the host (no
device): image.c against what the mathematics and the file formats fix.

Reference: NImage.reload (NImage.c:638-658), randomAugment / rotateCrop
(NImage.c:1016-1034, 551-572), bilinearInterpolate (NImage.c:146-158),
flip (NImage.c:355-370), distort / rgbToHsv / hsvToRgb (NImage.c:201-352),
resizeImage (NImage.c:474-530), loadImageAugmentPaths (ImageData.c:56-73),
fillTruthSmooth (ImageData.c:80-104), parseNetOption (NetworkFactory.c:
727-762)."""
import ctypes as C
import struct
import zlib

import numpy as np
import pytest

import aetcnn

RT = 5e-7  # the float RGB -> HSV -> RGB round trip: a few ulps of 1.0


def lib():
    return aetcnn.net_lib()


# ---- file decoding ------------------------------------------------------------
def _paeth(a, b, c):
    p = a + b - c
    pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
    if pa <= pb and pa <= pc:
        return a
    return b if pb <= pc else c


def png_bytes(pix, ctype, filters, palette=None, trns=None):
    """A PNG file (ISO/IEC 15948) of pix [H][W][bytes per pixel] uint8 with
    the given per-row filter types."""
    H, W, bpp = pix.shape
    raw = bytearray()
    prev = np.zeros(W * bpp, np.int64)
    for y in range(H):
        row = pix[y].reshape(-1).astype(np.int64)
        ft = filters[y % len(filters)]
        out = np.zeros_like(row)
        for i in range(row.size):
            a = row[i - bpp] if i >= bpp else 0
            b = prev[i] if y else 0
            c = prev[i - bpp] if (y and i >= bpp) else 0
            pred = [0, a, b, (a + b) // 2, _paeth(a, b, c)][ft]
            out[i] = (row[i] - pred) % 256
        raw += bytes([ft]) + bytes(out.astype(np.uint8))
        prev = row

    def chunk(t, data):
        return (struct.pack(">I", len(data)) + t + data +
                struct.pack(">I", zlib.crc32(t + data) & 0xFFFFFFFF))
    out = b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", W, H, 8, ctype, 0, 0, 0))
    if palette is not None:
        out += chunk(b"PLTE", bytes(palette.astype(np.uint8).reshape(-1)))
    if trns is not None:
        out += chunk(b"tRNS", bytes(trns.astype(np.uint8)))
    comp = zlib.compress(bytes(raw))
    out += chunk(b"IDAT", comp[:len(comp) // 2]) + chunk(b"IDAT", comp[len(comp) // 2:])
    return out + chunk(b"IEND", b"")


def planes(pix):
    return (np.transpose(pix, (2, 0, 1)).astype(np.float32) / np.float32(255))


@pytest.mark.parametrize("ctype,bpp", [(2, 3), (0, 1), (6, 4), (4, 2)])
def test_png_decode_every_filter(tmp_path, ctype, bpp):
    rng = np.random.default_rng(ctype)
    pix = rng.integers(0, 256, (7, 9, bpp), dtype=np.uint8)
    p = tmp_path / "a.png"
    p.write_bytes(png_bytes(pix, ctype, [0, 1, 2, 3, 4]))
    got = aetcnn.image_load(str(p), 9, 7, bpp)
    assert np.array_equal(got, planes(pix))


def test_png_palette(tmp_path):
    rng = np.random.default_rng(3)
    pal = rng.integers(0, 256, (16, 3))
    idx = rng.integers(0, 16, (5, 6, 1), dtype=np.uint8)
    p = tmp_path / "p.png"
    p.write_bytes(png_bytes(idx, 3, [4, 1], palette=pal))
    assert np.array_equal(aetcnn.image_load(str(p), 6, 5, 3), planes(pal[idx[..., 0]]))
    # with transparency the palette image has 4 channels (as stb_image reports)
    trns = rng.integers(0, 256, 16)
    p.write_bytes(png_bytes(idx, 3, [2], palette=pal, trns=trns))
    rgba = np.concatenate([pal, trns[:, None]], axis=1)
    assert np.array_equal(aetcnn.image_load(str(p), 6, 5, 4), planes(rgba[idx[..., 0]]))


def test_pnm_decode(tmp_path):
    rng = np.random.default_rng(4)
    pix = rng.integers(0, 256, (4, 5, 3), dtype=np.uint8)
    p = tmp_path / "a.ppm"
    p.write_bytes(b"P6\n# comment\n5 4\n255\n" + pix.tobytes())
    assert np.array_equal(aetcnn.image_load(str(p), 5, 4, 3), planes(pix))
    g = rng.integers(0, 256, (3, 2, 1), dtype=np.uint8)
    q = tmp_path / "a.pgm"
    q.write_bytes(b"P5 2 3 255\n" + g.tobytes())
    assert np.array_equal(aetcnn.image_load(str(q), 2, 3, 1), planes(g))


def test_decode_errors(tmp_path):
    """NImage.reload refuses images of another size or channel count."""
    pix = np.zeros((4, 4, 3), np.uint8)
    p = tmp_path / "a.png"
    p.write_bytes(png_bytes(pix, 2, [0]))
    for w, h, c in [(5, 4, 3), (4, 4, 1)]:
        with pytest.raises(aetcnn.HipError):
            aetcnn.image_load(str(p), w, h, c)
    bad = tmp_path / "b.png"
    data = bytearray(png_bytes(pix, 2, [0]))
    data[40:44] = b"\0\0\0\0"  # corrupt the compressed stream
    bad.write_bytes(bytes(data))
    with pytest.raises(aetcnn.HipError):
        aetcnn.image_load(str(bad), 4, 4, 3)
    with pytest.raises(aetcnn.HipError):
        aetcnn.image_load(str(tmp_path / "missing.png"), 4, 4, 3)
    (tmp_path / "x.jpg").write_bytes(b"\xff\xd8\xff\xe0" + bytes(100))
    with pytest.raises(aetcnn.HipError):
        aetcnn.image_load(str(tmp_path / "x.jpg"), 4, 4, 3)


def test_label_from_path():
    """fillTruthSmooth: exactly one label must occur in the path."""
    labels = ["airplane", "automobile", "bird", "cat"]
    assert aetcnn.label_from_path("train/123_cat.png", labels) == 3
    assert aetcnn.label_from_path("train/7_bird.png", labels) == 2
    assert aetcnn.label_from_path("train/7_dog.png", labels) == -1          # none
    assert aetcnn.label_from_path("train/cat_and_bird.png", labels) == -1   # two


# ---- the augmentation steps ---------------------------------------------------
def rotate_crop(src, rad, s, w, h, dx, dy, aspect):
    c, H, W = src.shape
    src = np.ascontiguousarray(src, np.float32)
    dst = np.empty((c, h, w), np.float32)
    lib().an_image_rotate_crop(src.ctypes.data, W, H, c, rad, s, w, h, dx, dy, aspect,
                               dst.ctypes.data)
    return dst


@pytest.mark.parametrize("dx,dy", [(0, 0), (3, -2), (-5, 4), (9, 0)])
def test_rotate_crop_integer_offsets_are_exact_index_maps(dx, dy):
    """No rotation, scale 1, aspect 1, integer offset: output (x, y) is input
    (x + dx, y + dy) exactly, zero outside the image."""
    rng = np.random.default_rng(abs(dx * 7 + dy))
    src = rng.random((3, 8, 8), dtype=np.float32)
    got = rotate_crop(src, 0.0, 1.0, 8, 8, dx, dy, 1.0)
    want = np.zeros_like(src)
    for y in range(8):
        for x in range(8):
            if 0 <= y + dy < 8 and 0 <= x + dx < 8:
                want[:, y, x] = src[:, y + dy, x + dx]
    assert np.array_equal(got, want)


def test_rotate_crop_zoom_is_bilinear():
    """Scale 2 on an 8x8 image: output x samples input x/2 + 2, so even
    columns copy a pixel and odd ones average two neighbours (the same for
    rows)."""
    rng = np.random.default_rng(9)
    src = rng.random((1, 8, 8), dtype=np.float32)
    got = rotate_crop(src, 0.0, 2.0, 8, 8, 0.0, 0.0, 1.0)
    s64 = src[0].astype(np.float64)
    for y in range(8):
        for x in range(8):
            ry, rx = y / 2 + 2, x / 2 + 2
            iy, ix = int(ry), int(rx)
            fy, fx = ry - iy, rx - ix
            v = ((1 - fy) * (1 - fx) * s64[iy, ix] + (1 - fy) * fx * s64[iy, ix + 1] +
                 fy * (1 - fx) * s64[iy + 1, ix] + fy * fx * s64[iy + 1, ix + 1])
            assert abs(got[0, y, x] - v) <= 2e-7, (y, x)


def test_rotate_crop_half_turn():
    """180 degrees about the centre of an even-sized image maps (x, y) to
    (W - x, H - y): a point reflection (cos and sin of pi within 1e-16)."""
    rng = np.random.default_rng(10)
    src = rng.random((2, 6, 6), dtype=np.float32)
    got = rotate_crop(src, np.pi, 1.0, 6, 6, 0.0, 0.0, 1.0)
    want = np.zeros_like(src)
    want[:, 1:, 1:] = src[:, ::-1, ::-1][:, :5, :5]
    assert np.abs(got - want).max() <= 1e-6


def test_flip_mirrors_rows():
    rng = np.random.default_rng(11)
    im = rng.random((3, 4, 7), dtype=np.float32)
    got = im.copy()
    lib().an_image_flip(got.ctypes.data, 7, 4, 3)
    assert np.array_equal(got, im[:, :, ::-1])


def distort(im, hue, sat, val):
    out = np.ascontiguousarray(im, np.float32).copy()
    lib().an_image_distort(out.ctypes.data, im.shape[2], im.shape[1], hue, sat, val)
    return out


def test_distort_neutral_leaves_pixels():
    """Hue shift 0, saturation 1, exposure 1: RGB -> HSV -> RGB returns each
    pixel (the round trip's float rounding, v*(1 - s) with s = delta/max,
    stays within a few ulps of 1.0)."""
    rng = np.random.default_rng(12)
    im = rng.random((3, 16, 16), dtype=np.float32)
    im[:, 0, 0] = [0.25, 0.25, 0.25]      # grey: saturation 0
    im[:, 0, 1] = 0.0                     # black: value 0
    assert np.abs(distort(im, 0.0, 1.0, 1.0) - im).max() <= RT


def test_distort_closed_forms():
    px = lambda r, g, b: np.array([r, g, b], np.float32).reshape(3, 1, 1)
    # hue + 0.5 turns pure red into cyan, pure green into magenta
    assert np.array_equal(distort(px(1, 0, 0), 0.5, 1, 1).ravel(), [0, 1, 1])
    assert np.array_equal(distort(px(0, 1, 0), 0.5, 1, 1).ravel(), [1, 0, 1])
    # saturation 0 gives the grey of the maximum channel (value)
    assert np.array_equal(distort(px(0.5, 0.25, 0.75), 0, 0, 1).ravel(), [0.75] * 3)
    # exposure scales a grey pixel and clamps at 1
    assert np.array_equal(distort(px(0.25, 0.25, 0.25), 0, 1, 2).ravel(), [0.5] * 3)
    assert np.array_equal(distort(px(0.75, 0.75, 0.75), 0, 1, 2).ravel(), [1.0] * 3)
    # hue shifts wrap around: -0.25 from hue 0.1 is hue 0.85
    im = distort(px(1, 0, 0), 1.0 / 6, 1, 1)  # red + 60 degrees = yellow
    assert np.array_equal(im.ravel(), [1, 1, 0])


def test_distort_matches_colorsys():
    """distort = rgbToHsv, scale S and V, shift H (one wrap), hsvToRgb, clamp
    to [0, 1] (NImage.c:201-323), recomputed in float64 with the standard
    library's HSV conversions (colorsys, the same textbook algorithm in its
    own arithmetic): random pixels and distortions, saturation and exposure
    beyond 1 included, within float32 rounding."""
    import colorsys
    rng = np.random.default_rng(21)
    for k in range(12):
        im = rng.random((3, 9, 11), dtype=np.float32)
        im[:, 0, :3] = rng.random(3, dtype=np.float32)[:, None]  # greys
        hue = float(rng.uniform(-0.5, 0.5))
        sat, val = float(rng.uniform(0.3, 1.8)), float(rng.uniform(0.3, 1.8))
        got = distort(im, hue, sat, val)
        want = np.empty_like(got, dtype=np.float64)
        for y in range(im.shape[1]):
            for x in range(im.shape[2]):
                h, s_, v = colorsys.rgb_to_hsv(*(float(c) for c in im[:, y, x]))
                s_, v = s_ * sat, v * val
                h += hue
                if h > 1:
                    h -= 1
                if h < 0:
                    h += 1
                want[:, y, x] = np.clip(colorsys.hsv_to_rgb(h, s_, v), 0, 1)
        assert np.abs(got - want).max() <= 2e-6, (k, np.abs(got - want).max())


def test_resize_closed_form():
    src = np.array([[[1.0, 3.0], [5.0, 9.0]]], np.float32)  # 1 x 2 x 2
    dst = np.empty((1, 3, 3), np.float32)
    assert lib().an_image_resize(src.ctypes.data, 2, 2, 1, 3, 3, dst.ctypes.data) == 0
    assert np.array_equal(dst[0], [[1, 2, 3], [3, 4.5, 6], [5, 7, 9]])
    same = np.empty_like(src)
    assert lib().an_image_resize(src.ctypes.data, 2, 2, 1, 2, 2, same.ctypes.data) == 0
    assert np.array_equal(same, src)
    # a one-pixel side samples row / column 0; bad sizes are refused
    one = np.empty((1, 1, 3), np.float32)
    assert lib().an_image_resize(src.ctypes.data, 2, 2, 1, 3, 1, one.ctypes.data) == 0
    assert np.array_equal(one[0, 0], [1, 2, 3])
    assert lib().an_image_resize(src.ctypes.data, 2, 2, 1, 0, 3, one.ctypes.data) < 0


# ---- the whole augmentation -----------------------------------------------------
def test_augment_identity_at_zero_jitter():
    """Crop side fixed at the image size, no rotation, aspect 1, no flip, no
    hue / saturation / exposure change: the image comes back (within the
    float rounding of the HSV round trip)."""
    rng = np.random.default_rng(13)
    src = rng.random((3, 32, 32), dtype=np.float32)
    a = aetcnn.Augment.defaults(32, min_crop=32, max_crop=32, flip=0)
    for i in range(5):
        got = aetcnn.augment_image(src, a, seed=1, batch_no=2, image=i)
        assert np.abs(got - src).max() <= RT
    one = src[:1].copy()  # one channel: no HSV step, exact
    assert np.array_equal(aetcnn.augment_image(one, a, 1, 2, 0), one)


def test_augment_flip_is_the_only_change():
    rng = np.random.default_rng(14)
    src = rng.random((1, 16, 16), dtype=np.float32)
    a = aetcnn.Augment.defaults(16, min_crop=16, max_crop=16, flip=1)
    flips = 0
    for i in range(200):
        got = aetcnn.augment_image(src, a, seed=5, batch_no=0, image=i)
        if np.array_equal(got, src):
            continue
        assert np.array_equal(got, src[:, :, ::-1]), i
        flips += 1
    assert 70 <= flips <= 130  # probability 1/2


def test_augment_is_a_function_of_seed_batch_image():
    rng = np.random.default_rng(15)
    src = rng.random((3, 24, 24), dtype=np.float32)
    a = aetcnn.Augment.defaults(24, angle=15, aspect=1.3, hue=0.1, saturation=1.5, exposure=1.5)
    x = aetcnn.augment_image(src, a, 7, 3, 4)
    assert np.array_equal(x, aetcnn.augment_image(src, a, 7, 3, 4))
    assert not np.array_equal(x, aetcnn.augment_image(src, a, 7, 3, 5))
    assert not np.array_equal(x, aetcnn.augment_image(src, a, 8, 3, 4))
    assert x.min() >= 0 and x.max() <= 1


def test_augment_zoom_range():
    """min_crop = max_crop = 2w zooms 2x: every output pixel is a bilinear
    blend of the input at x/2 + offset, the offset within +-w/4 (half of
    (2w - w) / 2 in input pixels), so a constant image stays constant except
    where the last row or column samples half a pixel past the border (a
    blend with the zero outside, as getPixelExtend gives)."""
    src = np.full((1, 16, 16), 0.625, np.float32)
    a = aetcnn.Augment.defaults(16, min_crop=32, max_crop=32, flip=0)
    for i in range(20):
        got = aetcnn.augment_image(src, a, 3, 0, i)
        assert np.abs(got[:, :15, :15] - 0.625).max() <= 1e-6, i
        assert got.min() >= 0.625 / 4 - 1e-6 and got.max() <= 0.625 + 1e-6, i


def test_cfg_augment_keys(tmp_path):
    p = tmp_path / "a.cfg"
    p.write_text("[net]\nbatch=4\nwidth=28\nheight=28\nchannels=3\n"
                 "angle=7\naspect=1.2\nhue=.1\nsaturation=1.5\nexposure=1.25\nflip=0\n"
                 "min_crop=30\nlabel_smooth_eps=0.1\n[convolutional]\nfilters=2\n")
    a = aetcnn.Augment()
    eps = C.c_float()
    assert lib().an_cfg_augment(str(p).encode(), C.byref(a), C.byref(eps)) == 0
    assert (a.min_crop, a.max_crop, a.flip) == (30, 56, 0)
    assert (a.angle, a.hue) == (np.float32(7), np.float32(0.1))
    assert (a.aspect, a.saturation, a.exposure) == (np.float32(1.2), 1.5, 1.25)
    assert eps.value == np.float32(0.1)
    p.write_text("[net]\nwidth=32\nheight=32\nchannels=3\n")
    assert lib().an_cfg_augment(str(p).encode(), C.byref(a), None) == 0
    assert (a.min_crop, a.max_crop, a.flip, a.angle, a.aspect) == (32, 64, 1, 0, 1)
    assert (a.hue, a.saturation, a.exposure) == (0, 1, 1)
