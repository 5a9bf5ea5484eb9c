"""Learning-rate policy and subdivisions (NNetwork.c:154-157, 215-246,
667-680, 762-805; NetworkFactory.c:763-823).

The oracle's getCurrentRate is pinned by values each policy's definition
fixes exactly (ramp midpoints, halvings, step boundaries, the sigmoid's
midpoint) and by the reference's size_t arithmetic below the sigmoid's step.
The host library's rate (computed on the CPU, no GPU needed) must equal the
oracle's.  Subdivisions are pinned by an identity: without batch-norm and
dropout, two minibatches of B with subdivisions = 2 give the same update as
one batch of 2B."""
import math

import numpy as np
import pytest

import aetcnn
import oracle_lib as O
from conftest import rel_err

LR = 0.1


def rate(policy, n, **kw):
    return O.lr_rate(policy, LR, n, **kw)


def test_constant_and_burn_in():
    for n in (0, 1, 7, 10 ** 6):
        assert rate(O.CONSTANT, n) == np.float32(LR)
    # burn_in ramp lr * (n/burn_in)^power, then the policy
    assert rate(O.CONSTANT, 50, burn_in=100, power=1) == np.float32(LR * 0.5)
    assert rate(O.CONSTANT, 50, burn_in=100, power=4) == np.float32(LR / 16)
    assert rate(O.CONSTANT, 0, burn_in=100, power=4) == 0.0
    assert rate(O.CONSTANT, 100, burn_in=100, power=4) == np.float32(LR)
    # the ramp applies before any policy
    assert rate(O.STEPS, 25, burn_in=100, power=1, steps=[10], scales=[0.5]) == \
        np.float32(LR * 0.25)


def test_step_steps_exp():
    for n, want in ((0, LR), (9, LR), (10, LR / 2), (19, LR / 2), (25, LR / 4)):
        assert rate(O.STEP, n, step=10, scale=0.5) == np.float32(want), n
    kw = dict(steps=[3, 7], scales=[0.5, 0.25])
    for n, want in ((0, LR), (2, LR), (3, LR / 2), (6, LR / 2), (7, LR / 8), (10 ** 5, LR / 8)):
        assert rate(O.STEPS, n, **kw) == np.float32(want), n
    assert rate(O.EXP, 0, gamma=0.5) == np.float32(LR)
    assert rate(O.EXP, 3, gamma=0.5) == np.float32(LR / 8)


def test_poly_sigmoid_random():
    assert rate(O.POLY, 50, power=1, max_batches=100) == np.float32(LR / 2)
    assert rate(O.POLY, 50, power=2, max_batches=100) == np.float32(LR / 4)
    assert rate(O.POLY, 100, power=1, max_batches=100) == 0.0
    assert rate(O.SIG, 50, gamma=0.1, step=50) == np.float32(LR / 2)
    assert math.isclose(rate(O.SIG, 60, gamma=0.1, step=50), LR / (1 + math.e), rel_tol=1e-6)
    # batch_num is size_t: below `step` the difference wraps to ~1.8e19
    assert rate(O.SIG, 40, gamma=0.1, step=50) == 0.0
    O.lib().or_rand_seed(9)
    assert rate(O.RANDOM, 5, power=0) == np.float32(LR)  # pow(r, 0) = 1
    O.lib().or_rand_seed(9)
    r = O.lib().or_rand_uniform(0, 1)
    O.lib().or_rand_seed(9)
    assert math.isclose(rate(O.RANDOM, 5, power=2), LR * r * r, rel_tol=1e-6)


CASES = [
    (O.CONSTANT, {}),
    (O.CONSTANT, dict(burn_in=40, power=4)),
    (O.STEP, dict(step=17, scale=0.3)),
    (O.STEPS, dict(steps=[5, 20, 60], scales=[0.1, 2.0, 0.05], burn_in=3, power=2)),
    (O.EXP, dict(gamma=0.97)),
    (O.POLY, dict(power=0.9, max_batches=150)),
    (O.SIG, dict(gamma=0.2, step=30)),
    (O.RANDOM, dict(power=1.5)),
]


@pytest.mark.parametrize("policy,kw", CASES)
def test_host_rate_matches_oracle(policy, kw):
    """an_rate (the C host library) against or_lr_rate over batch numbers
    0..199; both draw the random policy from the same glibc rand()."""
    net = aetcnn.Network(4, 8, 8, 3)
    args = dict(burn_in=0, power=4.0, gamma=1.0, scale=1.0, step=1, max_batches=0,
                steps=(), scales=())
    args.update(kw)
    net.hyper(LR, 0.9, 5e-4)
    net.policy(policy, **args)
    for n in range(200):
        O.lib().or_rand_seed(n)
        want = O.lr_rate(policy, LR, n, **args)
        aetcnn.net_lib().an_rand_seed(n)
        got = net.rate(n)
        same_nan = math.isnan(got) and math.isnan(want)  # poly past max_batches
        assert got == want or same_nan or math.isclose(got, want, rel_tol=1e-6), (n, got, want)
    net.close()


def test_policy_argument_errors():
    net = aetcnn.Network(4, 8, 8, 3)
    lib = aetcnn.net_lib()
    assert lib.an_set_policy(net.h, 7, 0, 4.0, 1.0, 1.0, 1, 0, 0, None, None) == aetcnn.ACH_EINVAL
    assert lib.an_set_policy(net.h, aetcnn.POLICY_STEPS, 0, 4.0, 1.0, 1.0, 1, 0, 0, None,
                             None) == aetcnn.ACH_EINVAL
    assert lib.an_set_policy(net.h, aetcnn.POLICY_STEP, 0, 4.0, 1.0, 1.0, 0, 0, 0, None,
                             None) == aetcnn.ACH_EINVAL
    assert lib.an_set_subdivisions(net.h, 0) == aetcnn.ACH_EINVAL
    net.close()


def _plain_net(batch, seed=4):
    """conv 3x3/8 + bias (no BN) leaky -> conv 1x1/5 linear -> avgpool -> softmax"""
    O.lib().or_rand_seed(seed)
    n = O.OracleNet(batch, 6, 6, 3)
    n.conv(8, 3, 1, 1, 7, 0)  # leaky
    n.conv(5, 1, 1, 0, 3, 0)  # linear
    n.avgpool()
    n.softmax()
    n.hyper(0.05, 0.9, 5e-4)
    n.finalize()
    return n


def test_oracle_subdivisions_equal_one_large_batch():
    rng = np.random.default_rng(3)
    B = 4
    x = rng.random((2 * B, 3, 6, 6), dtype=np.float32)
    truth = np.zeros((2 * B, 5), np.float32)
    truth[np.arange(2 * B), rng.integers(0, 5, 2 * B)] = 1
    big = _plain_net(2 * B)
    sub = _plain_net(B)
    sub.subdivisions(2)
    w0 = sub.buffer(0, 2).copy()
    sub.train(x[:B], truth[:B])
    assert np.array_equal(sub.buffer(0, 2), w0), "no update after the first minibatch"
    assert sub.iteration() == 0 and sub.seen() == B
    sub.train(x[B:], truth[B:])
    big.train(x, truth)
    assert sub.iteration() == big.iteration() == 1 and sub.seen() == big.seen() == 2 * B
    for i in (0, 1):
        for which in (2, 3, 4, 5):
            e = rel_err(sub.buffer(i, which), big.buffer(i, which))
            assert e < 1e-5, (i, which, e)
    # the second iteration updates again after two minibatches
    sub.train(x[:B], truth[:B])
    sub.train(x[B:], truth[B:])
    big.train(x, truth)
    assert rel_err(sub.buffer(0, 2), big.buffer(0, 2)) < 1e-5
    sub.close()
    big.close()


def test_oracle_update_uses_policy_rate():
    """Two nets, one with the constant rate lr/2 and one with STEPS halving lr
    at batch 1 (the first update sees batch_num = 1): identical parameters."""
    rng = np.random.default_rng(5)
    x = rng.random((4, 3, 6, 6), dtype=np.float32)
    truth = np.zeros((4, 5), np.float32)
    truth[np.arange(4), [0, 1, 2, 3]] = 1
    a, b = _plain_net(4), _plain_net(4)
    a.hyper(0.025, 0.9, 5e-4)
    b.hyper(0.05, 0.9, 5e-4)
    b.policy(O.STEPS, steps=[1], scales=[0.5])
    for _ in range(2):
        assert a.train(x, truth) == b.train(x, truth)
    assert np.array_equal(a.buffer(0, 2), b.buffer(0, 2))
    a.close()
    b.close()
