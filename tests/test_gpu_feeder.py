"""Input pipeline (an_feeder_*, ImageData.c:20-224): image-list and CIFAR-10
binary sources, sampling, the augmentation and label smoothing as documented
in aetcnn_net.h (each image equals an_augment_image of the decoded source
image, whose arithmetic is pinned on the CPU in test_augment.py); batches
arrive in order on the network stream while the copy overlaps the previous
step; training on fed batches equals training on the same host batches."""
import numpy as np
import pytest

import aetcnn
from aetcnn import configs

pytestmark = pytest.mark.gpu

M64 = (1 << 64) - 1


def mix64(z):
    z = np.uint64(z) if np.isscalar(z) else z.astype(np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def draw(seed, bn, i, salt):
    """an_feeder_sample(seed, bn, i, salt) restated (documented in aetcnn_net.h)"""
    i = np.asarray(i, dtype=np.uint64)
    with np.errstate(over="ignore"):
        base = np.uint64((seed + 0x9E3779B97F4A7C15 * (bn + 1)) & M64)
        return mix64(base + mix64(i * np.uint64(4) + np.uint64(salt)))


def tiny_net(batch):
    aetcnn.net_lib().an_rand_seed(1)
    B, h, w, c = configs.dims("tiny", batch)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, "tiny")
    net.finalize()
    return net


def device_input(net):
    ops = aetcnn.ops()
    lib = aetcnn.net_lib()
    ops.ach_stream_sync(net.stream)
    x = aetcnn.DeviceArray.wrap(lib.an_input(net.h), (net.batch, 3, 32, 32)).numpy(net.stream)
    t = aetcnn.DeviceArray.wrap(lib.an_truth(net.h), (net.batch, 10)).numpy(net.stream)
    return x, t


def test_sample_matches_documented_hash(gpu):
    lib = aetcnn.net_lib()
    for seed, bn, i, w in [(0, 0, 0, 0), (7, 3, 11, 1), (2**63 + 5, 99, 1234, 2)]:
        assert lib.an_feeder_sample(seed, bn, i, w) == int(draw(seed, bn, i, w))


def test_cifar_batches(gpu, tmp_path):
    rng = np.random.default_rng(0)
    recs = []
    files = []
    for n in (300, 200):
        r = rng.integers(0, 256, (n, 3073), dtype=np.uint8)
        r[:, 0] = rng.integers(0, 10, n)
        r[5, 0] = 200  # label outside the classes: skipped by the reader
        recs.append(np.delete(r, 5, axis=0))
        p = tmp_path / f"data_batch_{len(files)}.bin"
        p.write_bytes(r.tobytes())
        files.append(str(p))
    recs = np.concatenate(recs)
    net = tiny_net(8)
    seed, eps = 5, 0.1
    aug = aetcnn.Augment.defaults(32, angle=10, aspect=1.2, hue=0.1, saturation=1.5,
                                  exposure=1.5)
    feeder = aetcnn.Feeder(net, cifar_files=files, threads=3, seed=seed, augment=aug,
                           label_smooth_eps=eps)
    try:
        for bn in range(5):
            feeder.next()
            x, t = device_input(net)
            idx = draw(seed, bn, np.arange(8), 0) % np.uint64(len(recs))
            for i in range(8):
                r = recs[int(idx[i])]
                img = r[1:].reshape(3, 32, 32).astype(np.float32) / np.float32(255)
                assert np.array_equal(x[i], aetcnn.augment_image(img, aug, seed, bn, i)), (bn, i)
                want = np.full(10, eps / 9, np.float32)
                want[r[0]] = 1 - eps
                assert np.array_equal(t[i], want), (bn, i)
        assert feeder.served() == 5
    finally:
        feeder.close()
        net.close()


def synthetic_batch(seed, bn, batch, inputs, classes):
    j = np.arange(batch * inputs, dtype=np.uint64)
    x = ((draw(seed, bn, j, 2) >> np.uint64(40)).astype(np.float32) *
         np.float32(1.0 / 16777216.0)).reshape(batch, inputs)
    labels = (draw(seed, bn, np.arange(batch), 3) % np.uint64(classes)).astype(np.int64)
    t = np.zeros((batch, classes), np.float32)
    t[np.arange(batch), labels] = 1
    return x, t


def test_fed_training_equals_host_batches(gpu):
    """Ten steps enqueued back to back through the feeder (no host sync
    between them) give the same losses as feeding the same batches from the
    host: the copy of batch k+1 never overtakes step k's use of batch k."""
    a, b = tiny_net(16), tiny_net(16)
    feeder = aetcnn.Feeder(a, threads=4, seed=9)
    try:
        for bn in range(10):
            feeder.next()
            a.train_step()
        la = a.loss()
        for bn in range(10):
            x, t = synthetic_batch(9, bn, 16, 3 * 32 * 32, 10)
            lb = b.train(x.reshape(16, 3, 32, 32), t)
        assert la == lb
        for i in (0, 2, 4):
            assert np.array_equal(a.buffer(i, 2), b.buffer(i, 2))
    finally:
        feeder.close()
        a.close()
        b.close()


LABELS = [f"_c{k}_" for k in range(10)]


def write_png(path, pix):
    """8-bit RGB PNG (filter 0 rows) of pix [H][W][3]"""
    import struct
    import zlib
    H, W, _ = pix.shape
    raw = b"".join(b"\0" + pix[y].tobytes() for y in range(H))

    def chunk(t, d):
        return struct.pack(">I", len(d)) + t + d + struct.pack(">I", zlib.crc32(t + d))
    path.write_bytes(b"\x89PNG\r\n\x1a\n" +
                     chunk(b"IHDR", struct.pack(">IIBBBBB", W, H, 8, 2, 0, 0, 0)) +
                     chunk(b"IDAT", zlib.compress(raw)) + chunk(b"IEND", b""))


@pytest.mark.parametrize("fmt", ["png", "jpg"])
def test_paths_source(gpu, tmp_path, fmt):
    """An image list with labels from path substrings (the reference's
    training list and fillTruthSmooth): every fed image is the augmented
    decoded file, its truth the one-hot of the label in its name.  PNG and
    (4:2:0 baseline) JPEG files; a JPEG's decoded pixels are the host
    decoder's (an_image_load)."""
    rng = np.random.default_rng(1)
    (tmp_path / "train").mkdir()
    paths, pix = [], []
    for k in range(13):
        p = tmp_path / "train" / f"img{k}{LABELS[k % 10]}.{fmt}"
        img = rng.integers(0, 256, (32, 32, 3), dtype=np.uint8)
        if fmt == "png":
            write_png(p, img)
        else:
            from jpeg_writer import encode
            p.write_bytes(encode(img, quality=90, sampling=((2, 2), (1, 1), (1, 1)))[0])
            dec = aetcnn.image_load(str(p), 32, 32, 3)
            img = np.rint(np.transpose(dec, (1, 2, 0)) * 255).astype(np.uint8)
        paths.append(str(p))
        pix.append(img)
    lst = tmp_path / "train.list"
    lst.write_text("\n".join(paths) + "\n")
    net = tiny_net(8)
    seed = 21
    aug = aetcnn.Augment.defaults(32, angle=5, hue=0.05)
    feeder = aetcnn.Feeder(net, threads=2, seed=seed, augment=aug, paths_list=str(lst),
                           labels=LABELS)
    try:
        for bn in range(3):
            feeder.next()
            x, t = device_input(net)
            idx = draw(seed, bn, np.arange(8), 0) % np.uint64(len(paths))
            for i in range(8):
                k = int(idx[i])
                img = np.transpose(pix[k], (2, 0, 1)).astype(np.float32) / np.float32(255)
                assert np.array_equal(x[i], aetcnn.augment_image(img, aug, seed, bn, i)), (bn, i)
                want = np.zeros(10, np.float32)
                want[k % 10] = 1
                assert np.array_equal(t[i], want), (bn, i)
            net.train_step()
        assert np.isfinite(net.loss())
    finally:
        feeder.close()
        net.close()


def test_paths_source_errors(gpu, tmp_path):
    """A path with no label (or two) refuses the list at creation; a file that
    cannot be decoded makes an_feeder_next fail (the reference aborts)."""
    net = tiny_net(8)
    try:
        lst = tmp_path / "bad.list"
        lst.write_text(str(tmp_path / "x_nolabel.png") + "\n")
        with pytest.raises(aetcnn.HipError):
            aetcnn.Feeder(net, threads=1, paths_list=str(lst), labels=LABELS)
        lst.write_text(str(tmp_path / "missing_c1_.png") + "\n")
        f = aetcnn.Feeder(net, threads=1, paths_list=str(lst), labels=LABELS)
        with pytest.raises(aetcnn.HipError):
            f.next()
        f.close()
    finally:
        net.close()
