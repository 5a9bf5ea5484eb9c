"""NaN handling of the training step.  The reference's CPU path stops the
process where a NaN appears in batch normalisation (NormData.normalize exits
on a NaN normalized value, NormData.c:273-276) or in a BN layer's scales or
scale updates (ScaleData.addUpdatesToScale / scaleUpdates abort,
ScaleData.c:51-54, 67-70).  Here every step ends with one scan of those
arrays and the loss read returns ACH_ENAN naming the first array found."""
import numpy as np
import pytest

import aetcnn
from aetcnn import configs

pytestmark = pytest.mark.gpu


def tiny_net(batch=8):
    aetcnn.net_lib().an_rand_seed(1)
    B, h, w, c = configs.dims("tiny", batch)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, "tiny")
    net.finalize()
    return net


def test_nan_input_stops_at_first_bn_statistics(gpu):
    net = tiny_net()
    try:
        x, t, _ = configs.synthetic_batch("tiny", 5, 8)
        assert np.isfinite(net.train(x, t))
        assert net.nan_status() is None
        x[3, 1, 5, 7] = np.nan
        with pytest.raises(aetcnn.HipError, match=f"code {aetcnn.ACH_ENAN}"):
            net.train(x, t)
        # layer 0's mean (tag 0): the first normalize the reference runs
        assert net.nan_status() == (0, 0)
        with pytest.raises(aetcnn.HipError, match=f"code {aetcnn.ACH_ENAN}"):
            net.loss()  # sticky: the state now holds the NaN
    finally:
        net.close()


def test_nan_scale_stops_at_first_scale_update(gpu):
    """A NaN BN scale in layer 2 makes its output, the loss and every delta
    below NaN; the reference's update loop (NNetwork.updateCPU, layers in
    order) then aborts first in layer 0's addUpdatesToScale, which checks the
    scales and the scale updates.  The scan runs after the step's update,
    which has carried the NaN updates into layer 0's scales: (0, scales)."""
    net = tiny_net()
    try:
        x, t, _ = configs.synthetic_batch("tiny", 6, 8)
        net.train(x, t)
        s = net.buffer(2, 6)
        s[3] = np.nan
        net.set_buffer(2, 6, s)
        with pytest.raises(aetcnn.HipError, match=f"code {aetcnn.ACH_ENAN}"):
            net.train(x, t)
        assert net.nan_status() == (0, 2)
    finally:
        net.close()


def test_clean_training_has_no_nan_status(gpu):
    net = tiny_net(16)
    try:
        for step in range(5):
            x, t, _ = configs.synthetic_batch("tiny", 10 + step, 16)
            assert np.isfinite(net.train(x, t))
        assert net.nan_status() is None
    finally:
        net.close()
