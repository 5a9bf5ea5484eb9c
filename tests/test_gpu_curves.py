"""100-step training-loss curves of BASELINE configs 3 (darknet) and 4
(AlexNet) at batch 128 against the oracle's curves committed under
tests/golden/ (written by tests/golden/make_loss_curves.py): the same
weights (rand() after srand(1)), the same dropout masks and the same fresh
synthetic batch each step; |loss_gpu - loss_oracle| <= 1e-3 at every step."""
import json
import os

import numpy as np
import pytest

import aetcnn
from aetcnn import configs
from conftest import ROOT

GOLDEN = os.path.join(ROOT, "tests", "golden")


def load_curve(name):
    path = os.path.join(GOLDEN, f"{name}_b128_loss100.json")
    if not os.path.exists(path):
        pytest.skip(f"fixture {os.path.basename(path)} not generated")
    with open(path) as f:
        return json.load(f)


def test_curve_fixtures_well_formed():
    for name in ("darknet", "alexnet"):
        d = load_curve(name)
        assert d["config"] == name and d["batch"] == 128 and d["steps"] == 100
        losses = np.array(d["losses"])
        # labels are random, so the loss hovers around ln(10) rather than
        # falling; the curve must stay finite and in a sane range
        assert losses.shape == (100,) and np.all(np.isfinite(losses))
        assert np.all((losses > 0.1) & (losses < 20.0))


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["darknet", "alexnet"])
def test_loss_curve_100_steps(gpu, name):
    d = load_curve(name)
    aetcnn.net_lib().an_rand_seed(d["weight_seed"])
    B, h, w, c = configs.dims(name, d["batch"])
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, name)
    net.dropout_seed(d["dropout_seed"])
    net.finalize()
    worst, where = 0.0, -1
    try:
        for step, ref in enumerate(d["losses"]):
            x, truth, _ = configs.synthetic_batch(name, d["batch_seed"] + step, B)
            got = net.train(x, truth)
            err = abs(got - ref)
            if err > worst:
                worst, where = err, step
            assert err <= 1e-3, (name, step, got, ref)
    finally:
        net.close()
    print(f"{name} b128 100-step max |dloss| = {worst:.3g} at step {where}")


def test_oracle_reproduces_first_darknet_step(oracle):
    """The committed darknet curve matches the current oracle (first step)."""
    d = load_curve("darknet")
    L = oracle.lib()
    L.or_set_gemm_parallel(1)
    L.or_rand_seed(d["weight_seed"])
    B, h, w, c = configs.dims("darknet", d["batch"])
    onet = oracle.OracleNet(B, h, w, c)
    configs.build(onet, "darknet")
    onet.dropout_seed(d["dropout_seed"])
    onet.finalize()
    x, truth, _ = configs.synthetic_batch("darknet", d["batch_seed"], B)
    got = onet.train(x, truth)
    onet.close()
    assert abs(got - d["losses"][0]) <= 1e-6, (got, d["losses"][0])
