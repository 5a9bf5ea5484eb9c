"""Validation driver (an_validate_paths, Classifier.validateSingle,
Classifier.c:359-464) on the GPU: accuracies over an image list equal the
host composition of its steps (an_validation_image, an_predict, an_top_k),
with a partial last batch, an unlabelled path and images of other sizes
and channel counts; with topk clamped to every class, the top-k accuracy is
the labelled fraction exactly."""
import numpy as np
import pytest

import aetcnn
from aetcnn import configs
from test_augment import png_bytes

pytestmark = pytest.mark.gpu

LABELS = [f"_c{k}_" for k in range(10)]


def trained_tiny(batch=8, steps=3):
    aetcnn.net_lib().an_rand_seed(1)
    B, h, w, c = configs.dims("tiny", batch)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, "tiny")
    net.finalize()
    for s in range(steps):
        x, t, _ = configs.synthetic_batch("tiny", 40 + s, batch)
        net.train(x, t)
    return net


def image_list(tmp_path):
    rng = np.random.default_rng(2)
    sizes = [(32, 32, 3, 2), (40, 48, 3, 2), (64, 40, 1, 0), (36, 36, 4, 6), (50, 33, 3, 2)]
    paths = []
    for k in range(13):
        H, W, bpp, ctype = sizes[k % len(sizes)]
        pix = rng.integers(0, 256, (H, W, bpp), dtype=np.uint8)
        name = f"v{k}{LABELS[(3 * k) % 10]}.png" if k != 5 else "v5_nolabel.png"
        p = tmp_path / name
        p.write_bytes(png_bytes(pix, ctype, [0, 1]))
        paths.append(str(p))
    lst = tmp_path / "valid.list"
    lst.write_text("\n".join(paths) + "\n")
    return str(lst), paths


def test_validate_paths_matches_host_composition(gpu, tmp_path):
    net = trained_tiny()
    try:
        lst, paths = image_list(tmp_path)
        res = net.validate(lst, LABELS, topk=3)
        assert (res.images, res.unlabeled, res.topk) == (13, 1, 3)
        hit1 = hitk = 0
        for start in range(0, len(paths), 8):
            chunk = paths[start:start + 8]
            x = np.zeros((8, 3, 32, 32), np.float32)
            for i, p in enumerate(chunk):
                x[i] = aetcnn.validation_image(p, 32, 32, 3)
            out = net.predict(x)
            for i, p in enumerate(chunk):
                cls = next((j for j, lab in enumerate(LABELS) if lab in p), -1)
                idx = aetcnn.top_k(out[i], 3)
                hit1 += int(idx[0] == cls)
                hitk += int(cls in idx)
        assert res.top1_accuracy == np.float32(hit1) / np.float32(13)
        assert res.topk_accuracy == np.float32(hitk) / np.float32(13)
        every = net.validate(lst, LABELS, topk=50)
        assert every.topk == 10
        assert every.topk_accuracy == np.float32(12) / np.float32(13)
        assert every.top1_accuracy == res.top1_accuracy
    finally:
        net.close()


def test_validate_paths_errors(gpu, tmp_path):
    net = trained_tiny(steps=0)
    try:
        with pytest.raises(aetcnn.HipError):
            net.validate(str(tmp_path / "missing.list"), LABELS)
        lst = tmp_path / "bad.list"
        lst.write_text(str(tmp_path / "gone_c1_.png") + "\n")
        with pytest.raises(aetcnn.HipError):
            net.validate(str(lst), LABELS)
    finally:
        net.close()
