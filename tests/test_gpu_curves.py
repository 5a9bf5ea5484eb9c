"""100-step training-loss curves of BASELINE configs 3 (darknet) and 4
(AlexNet) at batch 128 against the oracle's curves committed under
tests/golden/ (written by tests/golden/make_loss_curves.py): the same
weights (rand() after srand(1)), the same dropout masks and the same fresh
synthetic batch each step."""
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


STRICT_STEPS = 6  # steps compared at |dloss| <= 1e-3 before divergence amplifies


def run_curve(name, d, perturb=False):
    aetcnn.net_lib().an_rand_seed(d["weight_seed"])
    B, h, w, c = configs.dims(name, d["batch"])
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, name)
    net.dropout_seed(d["dropout_seed"])
    net.finalize()
    if perturb:  # one weight of the first layer moved by one ulp
        wts = net.buffer(0, 2)
        wts[0] = np.nextafter(wts[0], np.float32(1))
        net.set_buffer(0, 2, wts)
    losses = []
    try:
        for step in range(d["steps"]):
            x, truth, _ = configs.synthetic_batch(name, d["batch_seed"] + step, B)
            losses.append(net.train(x, truth))
    finally:
        net.close()
    return np.array(losses)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["darknet", "alexnet"])
def test_loss_curve_100_steps(gpu, name):
    """Free-running SGD amplifies any rounding difference: moving ONE weight
    by one ulp makes this implementation diverge from itself by ~3e-3 within
    10 darknet steps (measured).  So the oracle's curve is matched at
    |dloss| <= 1e-3 over the first steps, and over all 100 steps the
    GPU-vs-oracle differences must stay inside the envelope of that
    one-ulp self-divergence (x3), with 10-step mean losses within 0.05."""
    d = load_curve(name)
    ref = np.array(d["losses"])
    got = run_curve(name, d)
    err = np.abs(got - ref)
    print(f"{name} b128 |dloss| first {STRICT_STEPS} steps max {err[:STRICT_STEPS].max():.3g}, "
          f"100 steps max {err.max():.3g} mean {err.mean():.3g}")
    assert np.all(err[:STRICT_STEPS] <= 1e-3), err[:STRICT_STEPS]
    if err.max() <= 1e-3:
        return
    env = np.abs(run_curve(name, d, perturb=True) - got)
    print(f"{name} one-ulp self-divergence: max {env.max():.3g} mean {env.mean():.3g}")
    assert err.max() <= 3 * env.max() + 1e-3
    assert err.mean() <= 3 * env.mean() + 1e-3
    win = lambda a: a.reshape(-1, 10).mean(axis=1)
    assert np.all(np.abs(win(got) - win(ref)) <= 0.05), (win(got), win(ref))


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
