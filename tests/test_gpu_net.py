"""Whole-network parity: the C host network driving the HIP kernels against
the oracle network (same construction order, same glibc rand() weight init,
same counter-based dropout masks, same synthetic batches)."""
import os

import numpy as np
import pytest

import aetcnn
from aetcnn import configs
from conftest import rel_err, ROOT

pytestmark = pytest.mark.gpu

TOL = 1e-4


def make_pair(oracle, name, batch, seed=1, dropout_seed=0x5eed):
    B, h, w, c = configs.dims(name, batch)
    aetcnn.net_lib().an_rand_seed(seed)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, name)
    net.dropout_seed(dropout_seed)
    net.finalize()
    oracle.lib().or_rand_seed(seed)
    onet = oracle.OracleNet(B, h, w, c)
    configs.build(onet, name)
    onet.dropout_seed(dropout_seed)
    onet.finalize()
    return net, onet


def conv_layers(onet):
    return [i for i in range(onet.n_layers()) if onet.info(i)[0] == 0]


def test_initial_weights_identical(gpu, oracle):
    net, onet = make_pair(oracle, "tiny", 8)
    for i in conv_layers(onet):
        assert np.array_equal(net.buffer(i, 2), onet.buffer(i, 2)), i
        assert np.array_equal(net.buffer(i, 4), onet.buffer(i, 4)), i
        if onet.buffer(i, 6) is not None:
            assert np.array_equal(net.buffer(i, 6), onet.buffer(i, 6)), i


@pytest.mark.parametrize("name,batch", [("tiny", 128), ("darknet", 8)])
def test_one_step_per_layer(gpu, oracle, name, batch):
    oracle.lib().or_set_gemm_parallel(1)
    net, onet = make_pair(oracle, name, batch)
    x, truth, _ = configs.synthetic_batch(name, 42, batch)
    net.set_input(x, truth)
    net.forward(1)
    net.backward()
    loss_ref = onet.forward_backward(x, truth)
    loss = net.loss()
    assert abs(loss - loss_ref) <= 1e-4 * max(1.0, abs(loss_ref)), (loss, loss_ref)
    for i in range(onet.n_layers()):
        kind = onet.info(i)[0]
        if kind == 3:  # dropout shares its input's buffers
            continue
        assert rel_err(net.buffer(i, 0), onet.buffer(i, 0)) < TOL, ("output", i)
        if i > 0:
            assert rel_err(net.buffer(i, 1), onet.buffer(i, 1)) < 5 * TOL, ("delta", i)
        if kind == 0:
            assert rel_err(net.buffer(i, 3), onet.buffer(i, 3)) < 5 * TOL, ("dW", i)
            su = onet.buffer(i, 7)
            if su is not None:
                assert rel_err(net.buffer(i, 7), su) < 5 * TOL, ("dgamma", i)
                assert rel_err(net.buffer(i, 8), onet.buffer(i, 8)) < TOL, ("rolling mean", i)
                assert rel_err(net.buffer(i, 9), onet.buffer(i, 9)) < TOL, ("rolling var", i)
            else:
                assert rel_err(net.buffer(i, 5), onet.buffer(i, 5)) < 5 * TOL, ("dbias", i)
        if kind == 1:
            a, b = net.buffer(i, 14), onet.buffer(i, 14)
            # untaught (not teacher-forced) indices may flip on fp near-ties
            assert np.mean(a != b) < 1e-4, ("argmax", i)
    net.update()
    onet.update()
    for i in conv_layers(onet):
        assert rel_err(net.buffer(i, 2), onet.buffer(i, 2)) < TOL, ("W after update", i)
    # predicted labels from the softmax output
    last = onet.n_layers() - 1
    p_gpu = net.buffer(last, 0).reshape(batch, -1).argmax(1)
    p_ref = onet.buffer(last, 0).reshape(batch, -1).argmax(1)
    assert np.mean(p_gpu != p_ref) <= 1.0 / batch


def test_tiny_loss_curve_100_steps(gpu, oracle):
    """Config 0 for 100 SGD steps on one fixed batch: |dloss| <= 1e-3 each step."""
    oracle.lib().or_set_gemm_parallel(1)
    net, onet = make_pair(oracle, "tiny", 128)
    x, truth, _ = configs.synthetic_batch("tiny", 7)
    worst = 0.0
    for step in range(100):
        l_gpu = net.train(x, truth)
        l_ref = onet.train(x, truth)
        worst = max(worst, abs(l_gpu - l_ref))
        assert abs(l_gpu - l_ref) <= 1e-3, (step, l_gpu, l_ref)
    print(f"tiny 100-step max |dloss| = {worst:.3g}, final loss {l_gpu:.5f}")


def test_darknet_few_steps_with_dropout(gpu, oracle):
    oracle.lib().or_set_gemm_parallel(1)
    net, onet = make_pair(oracle, "darknet", 8)
    for step in range(3):
        x, truth, _ = configs.synthetic_batch("darknet", 100 + step, 8)
        l_gpu = net.train(x, truth)
        l_ref = onet.train(x, truth)
        assert abs(l_gpu - l_ref) <= 1e-3, (step, l_gpu, l_ref)
    for i in conv_layers(onet):
        assert rel_err(net.buffer(i, 2), onet.buffer(i, 2)) < TOL, i


def test_cfg_file_drives_same_network(gpu, oracle):
    path = os.path.join(ROOT, "aet-cnn_amd", "cfg", "tiny.cfg")
    aetcnn.net_lib().an_rand_seed(1)
    a = aetcnn.Network.from_cfg(path)
    aetcnn.net_lib().an_rand_seed(1)
    B, h, w, c = configs.dims("tiny")
    b = aetcnn.Network(B, h, w, c)
    configs.build(b, "tiny")
    b.finalize()
    assert a.n_layers() == b.n_layers()
    x, truth, _ = configs.synthetic_batch("tiny", 3)
    for _ in range(2):
        assert a.train(x, truth) == b.train(x, truth)


def test_alexnet_forward_shapes_and_step(gpu, oracle):
    """AlexNet-style at batch 2: strided 11x11 conv, overlapping pools, FC as conv."""
    oracle.lib().or_set_gemm_parallel(1)
    net, onet = make_pair(oracle, "alexnet", 2)
    x, truth, _ = configs.synthetic_batch("alexnet", 5, 2)
    l_gpu = net.train(x, truth)
    l_ref = onet.train(x, truth)
    assert abs(l_gpu - l_ref) <= 1e-3 * max(1, abs(l_ref))
    for i in conv_layers(onet):
        assert rel_err(net.buffer(i, 2), onet.buffer(i, 2)) < TOL, i
