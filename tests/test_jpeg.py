"""The JPEG decoder of the input pipeline (host/jpeg.c) on the CPU.

The reference decodes its image lists with the vendored stb_image
(NImage.loadImage, NImage.c:587-623).  No JPEG files or decoder ship with the
reference or this image, so the files here come from the baseline writer in
tests/jpeg_writer.py, which also computes the decode T.81 fixes for them (a
float64 inverse DCT rounded to the nearest level, the triangle-filter 2x
chroma upsampling and the JFIF colour conversion).  The decoder must match
that decode to within one level (float rounding at exact .5 ties) and almost
everywhere exactly, and stay close to the source image.  A wrong zig-zag
order, Huffman table, DC prediction, restart handling, sampling geometry or
colour transform moves samples by tens of levels."""
import struct

import numpy as np
import pytest

import aetcnn
from jpeg_writer import encode, ideal_decode


def load(tmp_path, data, w, h, c, name="a.jpg"):
    p = tmp_path / name
    p.write_bytes(data)
    planes = aetcnn.image_load(str(p), w, h, c)  # [c][h][w] floats / 255
    out = np.rint(planes * 255).astype(np.int64)
    return out[0] if c == 1 else np.moveaxis(out, 0, -1)


def smooth_image(h, w, c, seed):
    """a smooth image with some texture (JPEG's regime), uint8"""
    rng = np.random.default_rng(seed)
    y, x = np.mgrid[0:h, 0:w]
    base = []
    for k in range(c):
        f = 96 + 80 * np.sin(x / (5.0 + 2 * k) + y / (7.0 + k)) + 30 * np.cos(y / 3.0 - k)
        base.append(f + rng.normal(0, 6, (h, w)))
    img = np.clip(np.stack(base, -1), 0, 255).astype(np.uint8)
    return img[..., 0] if c == 1 else img


def check_decode(got, info, src, mean_tol):
    ideal = ideal_decode(info).astype(np.int64)
    d = np.abs(got - ideal)
    assert d.max() <= 1, d.max()
    assert (d == 0).mean() >= 0.999, (d == 0).mean()
    assert np.abs(got - src.astype(np.int64)).mean() < mean_tol


CASES = [
    # (h, w, channels, sampling of Y (chroma 1x1), restart, interleaved, deep, quality)
    (16, 16, 1, (1, 1), 0, True, False, 90),
    (29, 37, 1, (1, 1), 3, True, True, 75),
    (32, 48, 3, (1, 1), 0, True, False, 95),    # 4:4:4
    (31, 45, 3, (2, 2), 0, True, False, 90),    # 4:2:0, partial MCUs
    (40, 33, 3, (2, 1), 2, True, False, 85),    # 4:2:2 with restarts every 2 MCUs
    (24, 40, 3, (2, 2), 5, False, True, 90),    # one scan per component, deep codes
    (17, 9, 3, (1, 2), 1, True, True, 60),      # 4:4:0, a restart after every MCU
]


@pytest.mark.parametrize("h,w,c,ys,restart,inter,deep,q", CASES)
def test_jpeg_decode_matches_t81(tmp_path, h, w, c, ys, restart, inter, deep, q):
    src = smooth_image(h, w, c, h * w + q)
    sampling = (ys, (1, 1), (1, 1))
    data, info = encode(src, quality=q, sampling=sampling, restart=restart, interleaved=inter,
                        deep=deep)
    if deep:  # some Huffman codes longer than the decoder's 9-bit lookup
        i = data.index(b"\xff\xc4")
        counts = data[i + 5:i + 21]
        assert any(counts[9:])
    got = load(tmp_path, data, w, h, c)
    # (subsampled chroma drops the source's per-channel noise)
    check_decode(got, info, src, mean_tol=4.0 if q >= 85 and ys == (1, 1) else 8.0)


def test_jpeg_adobe_rgb_and_16bit_tables(tmp_path):
    """RGB components (Adobe APP14 transform 0) are not colour-converted;
    16-bit quantisation tables (Pq = 1)."""
    src = smooth_image(24, 24, 3, 7)
    data, info = encode(src, quality=92, adobe_rgb=True, q16=True)
    got = load(tmp_path, data, 24, 24, 3)
    check_decode(got, info, src, mean_tol=4.0)


def test_jpeg_flat_colours_exact(tmp_path):
    """a flat colour survives exactly (DC only; the colour transform's
    round trip of a grey level is exact)"""
    src = np.full((16, 24, 3), 77, np.uint8)
    data, info = encode(src, quality=90, sampling=((2, 2), (1, 1), (1, 1)))
    assert np.array_equal(load(tmp_path, data, 24, 16, 3), np.full((16, 24, 3), 77))


def test_jpeg_validation_path_and_channel_conversion(tmp_path):
    """a greyscale JPEG read as 3 channels by the validation reader
    (stb_image's conversion: grey replicated)"""
    src = smooth_image(20, 20, 1, 3)
    data, info = encode(src, quality=95)
    p = tmp_path / "g.jpg"
    p.write_bytes(data)
    v = aetcnn.validation_image(str(p), 20, 20, 3)
    assert np.array_equal(v[0], v[1]) and np.array_equal(v[1], v[2])
    ideal = ideal_decode(info).astype(np.float32) / 255
    assert np.abs(v[0] - ideal).max() <= 1.5 / 255


def _with_sof(data, marker):
    i = data.index(b"\xff\xc0")
    return data[:i + 1] + bytes([marker]) + data[i + 2:]


def test_jpeg_refused_forms(tmp_path):
    """progressive, arithmetic and lossless frames, 12-bit samples, CMYK and
    truncated files fail with an error (nothing decoded)"""
    src = smooth_image(16, 16, 3, 1)
    data, _ = encode(src, quality=90)
    bad = [_with_sof(data, 0xC2), _with_sof(data, 0xC9), _with_sof(data, 0xC3),
           data[:len(data) // 2], data[:40]]
    i = data.index(b"\xff\xc0")
    twelve = bytearray(data)
    twelve[i + 4] = 12
    bad.append(bytes(twelve))
    sof4 = struct.pack(">BHHB", 8, 16, 16, 4) + b"".join(
        struct.pack(">BBB", k + 1, 0x11, 0) for k in range(4))
    bad.append(b"\xff\xd8" + b"\xff\xc0" + struct.pack(">H", len(sof4) + 2) + sof4 + b"\xff\xd9")
    for k, d in enumerate(bad):
        with pytest.raises(aetcnn.HipError):
            load(tmp_path, d, 16, 16, 3, name=f"bad{k}.jpg")


def test_jpeg_corrupt_bytes_never_crash(tmp_path):
    """single-byte corruptions anywhere in a file decode or fail cleanly
    (the decoder bounds every read; the run would abort otherwise)"""
    src = smooth_image(24, 32, 3, 5)
    data, _ = encode(src, quality=80, sampling=((2, 2), (1, 1), (1, 1)), restart=2)
    rng = np.random.default_rng(11)
    ok = failed = 0
    for k in range(300):
        d = bytearray(data)
        d[int(rng.integers(2, len(d)))] = int(rng.integers(0, 256))
        try:
            load(tmp_path, bytes(d), 32, 24, 3, name="c.jpg")
            ok += 1
        except aetcnn.HipError:
            failed += 1
    assert ok + failed == 300
