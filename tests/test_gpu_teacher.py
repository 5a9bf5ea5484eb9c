"""Per-step parity along the reference's whole training trajectory.

Free-running SGD amplifies any rounding difference (test_gpu_curves.py), so
the 100-step loss bar is shown by teacher forcing: before every step the GPU
network takes the oracle's complete training state -- weights, biases, BN
scales, their momentum buffers and the rolling statistics (the iteration,
hence the dropout masks, already agrees) -- and both networks then train on
the same fresh batch.  Each step's loss must agree within 1e-3 and the
updated parameters within 1e-4 normwise relative (NNetwork.train,
NNetwork.c:740-805; ConvolutionalLayer.update, ConvolutionalLayer.c:959-980).

Config 3 (darknet-style) runs all 100 steps at batch 128, in ten tests of ten
steps that share one pair of networks, so progress shows per ten steps;
config 4 (AlexNet-style) runs 5 steps at batch 128."""
import numpy as np
import pytest

import aetcnn
from aetcnn import configs
from conftest import rel_err

pytestmark = pytest.mark.gpu

LOSS_TOL = 1e-3
PARAM_TOL = 1e-4
# weights, weight momenta, biases, bias momenta, scales, scale momenta,
# rolling mean, rolling variance
STATE_CODES = (2, 3, 4, 5, 6, 7, 8, 9)
PARAM_CODES = (2, 4, 6)
DARKNET_STEPS = 100
CHUNK = 10
BATCH_SEED = 2000


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


def param_layers(onet):
    return [i for i in range(onet.n_layers()) if onet.info(i)[0] == 0]


def bias_truth(onet, i, b0, v0, lr, batch):
    """float64 biases after the step of a conv layer without BN: b0 + lr/B *
    (v0 + sum of its final delta over images and positions) -- the update
    (ConvolutionalLayer.c:959-980) of the bias gradient (BiasData.c:40-57)
    in exact arithmetic, from the oracle's delta of the step."""
    F = b0.size
    d = onet.buffer(i, 1).reshape(batch, F, -1).astype(np.float64)
    db = d.sum(axis=(0, 2))
    return b0.astype(np.float64) + lr / batch * (v0.astype(np.float64) + db)


def teacher_step(net, onet, name, step, batch):
    """One teacher-forced step; returns (|dloss|, worst parameter error).
    Biases of layers without BN are a plain sum of ~10^5 deltas that cancel
    to a small total; where GPU and oracle differ by more than the bar there,
    both are judged against float64 arithmetic (the GPU within the bar, and
    no further from the oracle than the oracle is from float64), as for the
    BN weight gradients in test_gpu_net.py."""
    layers = param_layers(onet)
    pre = {}
    for i in layers:
        for code in STATE_CODES:
            v = onet.buffer(i, code)
            if v is not None and v.size:
                net.set_buffer(i, code, v)
                pre[(i, code)] = v
    x, truth, _ = configs.synthetic_batch(name, BATCH_SEED + step, batch)
    l_gpu = net.train(x, truth)
    l_ref = onet.train(x, truth)
    dl = abs(l_gpu - l_ref)
    assert dl <= LOSS_TOL, (name, step, l_gpu, l_ref)
    assert net.iteration() == onet.iteration() == step + 1
    worst = 0.0
    lr = configs.CONFIGS[name]["lr"]
    for i in layers:
        for code in PARAM_CODES:
            v = onet.buffer(i, code)
            if v is None or not v.size:
                continue
            got = net.buffer(i, code)
            e = rel_err(got, v)
            if e >= PARAM_TOL and code == 4 and onet.buffer(i, 6) is None:
                exact = bias_truth(onet, i, pre[(i, 4)], pre[(i, 5)], lr, batch)
                e_gpu, e_ref = rel_err(got, exact), rel_err(v, exact)
                print(f"{name} step {step} layer {i} biases: gpu-oracle {e:.2g}, "
                      f"gpu-f64 {e_gpu:.2g}, oracle-f64 {e_ref:.2g}")
                assert e_gpu < PARAM_TOL and e <= e_ref + PARAM_TOL, (name, step, i, e, e_gpu,
                                                                      e_ref)
                e = e_gpu
            worst = max(worst, e)
            assert e < PARAM_TOL, (name, step, i, code, e)
    return dl, worst


@pytest.fixture(scope="module")
def darknet_run(gpu, oracle):
    oracle.lib().or_set_gemm_parallel(1)
    net, onet = make_pair(oracle, "darknet", 128)
    run = dict(net=net, onet=onet, done=0, dloss=[], perr=[])
    yield run
    net.close()
    onet.close()


@pytest.mark.parametrize("chunk", range(DARKNET_STEPS // CHUNK))
def test_darknet_teacher_forced_100_steps(darknet_run, chunk):
    """Steps [10*chunk, 10*chunk + 10) of config 3 at batch 128 (a test run
    alone first replays the earlier steps of the trajectory)."""
    r = darknet_run
    end = (chunk + 1) * CHUNK
    while r["done"] < end:
        dl, pe = teacher_step(r["net"], r["onet"], "darknet", r["done"], 128)
        r["dloss"].append(dl)
        r["perr"].append(pe)
        r["done"] += 1
    dl = np.array(r["dloss"][end - CHUNK:end])
    pe = np.array(r["perr"][end - CHUNK:end])
    print(f"darknet b128 teacher-forced steps {end - CHUNK}-{end - 1}: max |dloss| "
          f"{dl.max():.3g}, max parameter error {pe.max():.3g}; over steps 0-{end - 1}: "
          f"max |dloss| {max(r['dloss']):.3g}")


def test_alexnet_teacher_forced_steps(gpu, oracle):
    """Config 4 at batch 128: 5 teacher-forced steps (strided 11x11 conv,
    5x5 conv, overlapping 3x3 pools, FC layers, dropout)."""
    oracle.lib().or_set_gemm_parallel(1)
    net, onet = make_pair(oracle, "alexnet", 128)
    dls, pes = [], []
    try:
        for step in range(5):
            dl, pe = teacher_step(net, onet, "alexnet", step, 128)
            dls.append(dl)
            pes.append(pe)
    finally:
        net.close()
        onet.close()
    print(f"alexnet b128 teacher-forced 5 steps: |dloss| {[f'{v:.2g}' for v in dls]}, "
          f"max parameter error {max(pes):.3g}")
