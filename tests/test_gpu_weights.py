"""darknet .weights save/load (NNetwork.c:64-151, ConvolutionalLayer.c:422-486):
byte layout against the reference's writer order, round trip into a fresh
network, the reference's tolerance of a truncated file, and the per-layer
load options dontload / dontloadscales / flipped and transposed headers."""
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


def tiny_with_options(seed, **layer_opts):
    """tiny net at batch 8; layer_opts maps layer index -> an_layer_options"""
    aetcnn.net_lib().an_rand_seed(seed)
    B, h, w, c = configs.dims("tiny", 8)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, "tiny")
    for i, o in layer_opts.items():
        net.set_layer_options(int(i[1:]), **o)
    net.finalize()
    return net


def _file(tmp_path, name, header, arrays):
    p = tmp_path / name
    p.write_bytes(np.array(header, np.int32).tobytes() + np.array([0], np.uint64).tobytes() +
                  b"".join(np.ascontiguousarray(a, np.float32).tobytes() for a in arrays))
    return str(p)


def test_load_dontload_and_dontloadscales(gpu, tmp_path):
    """dontload: the layer is skipped without reading (NNetwork.c:93-94), so
    the next layer reads the arrays that follow the header; dontloadscales:
    a BN layer reads biases then weights, no BN arrays
    (ConvolutionalLayer.c:461-482)."""
    net = tiny_with_options(3, l0=dict(dontload=1), l2=dict(dontloadscales=1))
    rng = np.random.default_rng(1)
    before = {c: net.buffer(0, c).copy() for c in (WEIGHTS, BIASES, SCALES)}
    before2 = {c: net.buffer(2, c).copy() for c in (SCALES, RMEAN, RVAR)}
    b2 = rng.standard_normal(32).astype(np.float32)
    w2 = rng.standard_normal(net.buffer(2, WEIGHTS).size).astype(np.float32)
    b4 = rng.standard_normal(10).astype(np.float32)
    w4 = rng.standard_normal(net.buffer(4, WEIGHTS).size).astype(np.float32)
    net.load_weights(_file(tmp_path, "a.weights", [0, 2, 5], [b2, w2, b4, w4]))
    for c, v in before.items():
        assert np.array_equal(net.buffer(0, c), v), c
    assert np.array_equal(net.buffer(2, BIASES), b2) and np.array_equal(net.buffer(2, WEIGHTS), w2)
    for c, v in before2.items():
        assert np.array_equal(net.buffer(2, c), v), c
    assert np.array_equal(net.buffer(4, BIASES), b4) and np.array_equal(net.buffer(4, WEIGHTS), w4)
    net.close()


def test_load_flipped(gpu, tmp_path):
    """flipped: the weights read are [C*k*k][n] and transposed to [n][C*k*k]
    (ConvolutionalLayer.c:483-485, transposeMatrix :443-453)."""
    net = tiny_with_options(3, l4=dict(flipped=1))
    rng = np.random.default_rng(2)
    arrays, want = [], {}
    for i in (0, 2, 4):
        n = net.buffer(i, BIASES).size
        k = net.buffer(i, WEIGHTS).size // n
        bn = i != 4
        b = rng.standard_normal(n).astype(np.float32)
        bn_arr = [rng.standard_normal(n).astype(np.float32) for _ in range(3)] if bn else []
        w = rng.standard_normal((k, n) if i == 4 else (n, k)).astype(np.float32)
        arrays += [b] + bn_arr + [w]
        want[i] = w.T.copy() if i == 4 else w
    net.load_weights(_file(tmp_path, "f.weights", [0, 2, 5], arrays))
    for i in (0, 2, 4):
        assert np.array_equal(net.buffer(i, WEIGHTS), want[i].ravel()), i
    net.close()


def test_load_transposed_connected(gpu, tmp_path):
    """A header with major or minor above 1000 marks darknet's transposed
    files: connected layers' weights [inputs][outputs] are transposed on load
    (darknet's load_connected_weights; the reference computes the flag at
    NNetwork.c:90); convolutional layers are read as they are."""
    aetcnn.net_lib().an_rand_seed(1)
    B, h, w, c = configs.dims("fcnet", 16)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, "fcnet")
    net.finalize()
    rng = np.random.default_rng(4)
    arrays, want = [], {}
    for i in (0, 2, 4):  # conv (BN), connected (BN), connected
        n = net.buffer(i, BIASES).size
        k = net.buffer(i, WEIGHTS).size // n
        bn = i != 4
        b = rng.standard_normal(n).astype(np.float32)
        bn_arr = [rng.standard_normal(n).astype(np.float32) for _ in range(3)] if bn else []
        if i == 0:
            wts = rng.standard_normal((n, k)).astype(np.float32)
            arrays += [b] + bn_arr + [wts]
            want[i] = wts
        else:  # darknet connected order: biases, weights, BN arrays
            wts = rng.standard_normal((k, n)).astype(np.float32)
            arrays += [b, wts] + bn_arr
            want[i] = wts.T.copy()
    net.load_weights(_file(tmp_path, "t.weights", [0, 1001, 0], arrays))
    for i in (0, 2, 4):
        assert np.array_equal(net.buffer(i, WEIGHTS), want[i].ravel()), i
    net.close()
