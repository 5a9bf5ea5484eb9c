"""darknet .weights save/load (NNetwork.c:64-151, ConvolutionalLayer.c:422-486):
byte layout against the reference's writer order, round trip into a fresh
network, and the reference's tolerance of a truncated file."""
import numpy as np
import pytest

import aetcnn
from aetcnn import configs

pytestmark = pytest.mark.gpu

# an_layer_buffer codes
WEIGHTS, BIASES, SCALES, RMEAN, RVAR = 2, 4, 6, 8, 9


def trained_tiny(seed, steps):
    aetcnn.net_lib().an_rand_seed(seed)
    B, h, w, c = configs.dims("tiny", 8)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, "tiny")
    net.finalize()
    for s in range(steps):
        x, truth, _ = configs.synthetic_batch("tiny", 50 + s, B)
        net.train(x, truth)
    return net


def conv_ids(net):
    return [i for i in range(net.n_layers()) if net.shape(i)[0] == 0]


def expected_bytes(net):
    """saveWeightsUpto: int32 {0, 2, 5}, uint64 seen = iteration*batch, then
    per conv layer biases, [scales, rolling mean, rolling variance], weights."""
    parts = [np.array([0, 2, 5], np.int32).tobytes(),
             np.array([net.iteration() * 8], np.uint64).tobytes()]
    for i in conv_ids(net):
        bn = net.buffer(i, SCALES) is not None and net.buffer(i, SCALES).size > 0
        arrays = [BIASES] + ([SCALES, RMEAN, RVAR] if bn else []) + [WEIGHTS]
        parts += [net.buffer(i, a).astype(np.float32).tobytes() for a in arrays]
    return b"".join(parts)


def test_weights_file_layout(gpu, tmp_path):
    net = trained_tiny(1, 3)
    p = tmp_path / "tiny.weights"
    net.save_weights(str(p))
    assert p.read_bytes() == expected_bytes(net)
    net.close()


def test_weights_round_trip(gpu, tmp_path):
    a = trained_tiny(1, 3)
    p = tmp_path / "a.weights"
    a.save_weights(str(p))
    b = trained_tiny(7, 0)  # different initial weights
    b.load_weights(str(p))
    assert b.seen() == a.iteration() * 8 and b.iteration() == a.iteration()
    for i in conv_ids(a):
        for code in (WEIGHTS, BIASES, SCALES, RMEAN, RVAR):
            x, y = a.buffer(i, code), b.buffer(i, code)
            if x is None or x.size == 0:
                continue
            assert np.array_equal(x, y), (i, code)
    # same parameters, iteration (dropout masks) and batch -> same forward loss
    x, truth, _ = configs.synthetic_batch("tiny", 99, 8)
    assert a.train(x, truth) == b.train(x, truth)
    a.close()
    b.close()


def test_truncated_weights_file(gpu, tmp_path):
    a = trained_tiny(1, 1)
    p = tmp_path / "a.weights"
    a.save_weights(str(p))
    data = p.read_bytes()
    first = conv_ids(a)[0]
    # keep the header and the first layer's biases + half of its scales
    n0 = a.buffer(first, BIASES).size
    cut = 20 + 4 * n0 + 4 * (n0 // 2)
    q = tmp_path / "short.weights"
    q.write_bytes(data[:cut])
    b = trained_tiny(7, 0)
    before = {c: b.buffer(first, c).copy() for c in (SCALES, WEIGHTS)}
    b.load_weights(str(q))
    assert np.array_equal(b.buffer(first, BIASES), a.buffer(first, BIASES))
    got = b.buffer(first, SCALES)
    assert np.array_equal(got[:n0 // 2], a.buffer(first, SCALES)[:n0 // 2])
    assert np.array_equal(got[n0 // 2:], before[SCALES][n0 // 2:])
    assert np.array_equal(b.buffer(first, WEIGHTS), before[WEIGHTS])
    a.close()
    b.close()
