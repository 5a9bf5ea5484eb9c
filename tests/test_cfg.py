"""The darknet .cfg parser, key by key, without a device
(an_parse_cfg_unfinalized builds the layers on the host only), and the
oracle's restatement of the per-layer options the reference's CPU path acts
on (stopbackward, onlyforward, learning_rate), pinned on the CPU.

Reference: NetworkFactory.c:77-173 (createConvolutional), 543-601 (pools,
softmax), 656-663 and 926-935 (per-layer options), 881-893 and 981-991
(stopbackward freezes the layers below), 671-823 (parseNetOption);
NNetwork.c:627-654 (backward loop), 667-680 (updateCPU);
ConvolutionalLayer.c:959-960 (learning_rate_scale)."""
import numpy as np
import pytest

import aetcnn
from aetcnn import configs

NET = "[net]\nbatch=4\nheight=8\nwidth=8\nchannels=3\nlearning_rate=0.01\n"
CONV = "[convolutional]\nfilters=4\nsize=3\npad=1\nactivation=leaky\n"
TAIL = "[avgpool]\n[softmax]\n"


def parse(tmp_path, text, name="t.cfg"):
    p = tmp_path / name
    p.write_text(text)
    try:
        return aetcnn.Network.from_cfg(str(p), finalize=False)
    except ValueError:
        return None


def opts(net, i):
    return net.layer_options(i)


def test_layer_options_parsed(tmp_path):
    net = parse(tmp_path, NET + CONV + "stopbackward=1\nflipped=1\nlearning_rate=0.5\n" +
                "[maxpool]\nsize=2\nstride=2\nonlyforward=1\ndontload=1\n" +
                CONV + "batch_normalize=1\ndontloadscales=1\n" + TAIL)
    assert net is not None
    o = opts(net, 0)
    assert o["stopbackward"] == 1 and o["flipped"] == 1 and o["onlyforward"] == 0
    assert o["learning_rate_scale"] == np.float32(0.5)
    o = opts(net, 1)
    assert o["onlyforward"] == 1 and o["dontload"] == 1 and o["stopbackward"] == 0
    assert opts(net, 2)["dontloadscales"] == 1
    assert opts(net, 2)["learning_rate_scale"] == 1.0
    net.close()


def test_layer_options_default(tmp_path):
    net = parse(tmp_path, NET + CONV + TAIL)
    assert opts(net, 0) == dict(stopbackward=0, onlyforward=0, dontload=0, dontloadscales=0,
                                flipped=0, learning_rate_scale=1.0)
    net.close()


def test_flipped_only_on_convolutional(tmp_path):
    net = parse(tmp_path, NET + CONV + "[maxpool]\nsize=2\nstride=2\nflipped=1\n" + TAIL)
    assert net is not None and opts(net, 1)["flipped"] == 0  # unused field of a pool
    net.close()


# (keys, stride_x, stride_y) as createConvolutional resolves them
# (NetworkFactory.c:83-90): a missing or nonpositive one falls back to stride
@pytest.mark.parametrize("keys,sx,sy", [
    ("stride_x=2\nstride_y=2\n", 2, 2),
    ("stride=2\n", 2, 2),
    ("stride_x=2\nstride_y=1\n", 2, 1),
    ("stride_x=2\n", 2, 1),                      # stride_y falls back to stride = 1
    ("stride=2\nstride_x=2\n", 2, 2),            # stride_y falls back to stride = 2
    ("stride=3\nstride_y=0\nstride_x=1\n", 1, 3),
])
def test_conv_stride_xy(tmp_path, keys, sx, sy):
    net = parse(tmp_path, NET + "[convolutional]\nfilters=4\nsize=3\npad=1\n" + keys + TAIL)
    assert net is not None
    assert net.shape(0)[2:4] == [(8 + 2 - 3) // sy + 1, (8 + 2 - 3) // sx + 1]
    net.close()


# (keys, out_h, out_w) on the 8x8 conv output, createMaxPool's keys
# (NetworkFactory.c:544-547): stride_x / stride_y default to stride, size to
# the stride key, padding to size - 1
@pytest.mark.parametrize("keys,oh,ow", [
    ("size=2\nstride_x=2\nstride_y=2\n", 4, 4),
    ("size=2\nstride=2\nstride_y=1\n", 8, 4),
    ("stride_x=2\nstride_y=3\n", 3, 4),         # size 1 (the stride key), padding 0
    ("size=3\nstride=1\nstride_x=2\n", 8, 4),
])
def test_maxpool_stride_xy(tmp_path, keys, oh, ow):
    net = parse(tmp_path, NET + CONV + "[maxpool]\n" + keys + TAIL)
    assert net is not None and net.shape(1)[2:4] == [oh, ow]
    net.close()
    assert parse(tmp_path, NET + CONV + "[maxpool]\nsize=2\nstride_x=0\n" + TAIL) is None


@pytest.mark.parametrize("section,key", [
    (CONV, "share_index=0"), (CONV, "share_index=-1"), (CONV, "assisted_excitation=1"),
    (CONV, "sway=1"), (CONV, "rotate=1"), (CONV, "stretch=1"), (CONV, "stretch_sway=1"),
    (CONV, "bin_output=1"), (CONV, "groups=2"), (CONV, "dilation=2"), (CONV, "xnor=1"),
    (CONV, "binary=1"), (CONV, "antialiasing=1"), (CONV, "cbn=1"),
    ("[maxpool]\nsize=2\nstride=2\n", "maxpool_depth=1"),
    ("[dropout]\nprobability=0.5\n", "dropblock=1"),
])
def test_unbuilt_keys_rejected(tmp_path, section, key):
    assert parse(tmp_path, NET + CONV + section + key + "\n" + TAIL) is None


@pytest.mark.parametrize("key", ["spatial=1", "noloss=1", "tree=data/tree.txt"])
def test_softmax_keys_rejected(tmp_path, key):
    assert parse(tmp_path, NET + CONV + "[avgpool]\n[softmax]\n" + key + "\n") is None


def test_net_keys(tmp_path):
    assert parse(tmp_path, NET + "time_steps=2\n" + CONV + TAIL) is None
    assert parse(tmp_path, NET + "inputs=100\n" + CONV + TAIL) is None
    net = parse(tmp_path, NET + "inputs=192\n" + CONV + TAIL)
    assert net is not None
    net.close()


def test_dilation_ignored_for_1x1(tmp_path):
    """createConvolutional forces dilation = 1 for size 1 (NetworkFactory.c:97-98)"""
    net = parse(tmp_path, NET + "[convolutional]\nfilters=4\nsize=1\ndilation=2\n" + TAIL)
    assert net is not None
    net.close()


def test_cpu_path_no_op_keys_accepted(tmp_path, capfd):
    """Keys the reference reads but its CPU training step never acts on."""
    net = parse(tmp_path, NET + "adam=1\nloss_scale=128\nhue=.1\nsaturation=1.5\n" + CONV +
                "dontsave=1\nclip=1\ntrain_only_bn=1\ndont_update=5\nburnin_update=2\n"
                "coordconv=1\ndot=1\ngrad_centr=1\nstream=1\n" + TAIL)
    assert net is not None
    net.close()
    assert "unused field" not in capfd.readouterr().err


def test_unknown_keys_reported(tmp_path, capfd):
    net = parse(tmp_path, NET + "bogus_net_key=3\n" + CONV + "bogus=1\n" + TAIL)
    assert net is not None
    net.close()
    err = capfd.readouterr().err
    assert "unused field [net] bogus_net_key=3" in err
    assert "unused field [convolutional] bogus=1" in err


def test_shipped_cfgs_parse_without_warnings(capfd):
    import os
    from conftest import ROOT
    for name in ("tiny", "darknet", "alexnet"):
        net = aetcnn.Network.from_cfg(os.path.join(ROOT, "aet-cnn_amd", "cfg", f"{name}.cfg"),
                                      finalize=False)
        assert net.n_layers() == len(configs.CONFIGS[name]["layers"])
        net.close()
    assert "unused" not in capfd.readouterr().err


def test_set_layer_options_host_api():
    net = aetcnn.Network(2, 8, 8, 3)
    net.conv(4, 3, 1, 1, aetcnn.LEAKY, 1)
    net.maxpool(2, 2, 1)
    net.set_layer_options(0, learning_rate_scale=0.25, onlyforward=1)
    assert net.layer_options(0)["learning_rate_scale"] == 0.25
    with pytest.raises(aetcnn.HipError):
        net.set_layer_options(1, flipped=1)   # flipped is a conv-layer option
    net.close()


# ---- the oracle's restatement of the options, pinned on the CPU ---------------

def _tiny_pair(oracle, tweak):
    """Two oracle tiny nets (seed 1); tweak(i, net) sets options on one."""
    nets = []
    for k in range(2):
        oracle.lib().or_rand_seed(1)
        n = oracle.OracleNet(*configs.dims("tiny", 8))
        configs.build(n, "tiny")
        if k:
            tweak(n)
        n.finalize()
        nets.append(n)
    return nets


def test_oracle_stopbackward_freezes_layers_below(oracle):
    """stopbackward on layer 2 (second conv): the backward loop stops before
    it, so its own update is the decay term alone and the conv layer below
    is frozen (train = 0): after one step its weights and momenta are those
    of initialisation, while the untouched network moves them."""
    plain, stop = _tiny_pair(oracle, lambda n: n.set_layer_options(2, stopbackward=1))
    x, t, _ = configs.synthetic_batch("tiny", 3, 8)
    w0 = {i: stop.buffer(i, 2).copy() for i in (0, 2, 4)}
    plain.train(x, t)
    stop.train(x, t)
    assert np.array_equal(stop.buffer(0, 2), w0[0])
    assert not np.any(stop.buffer(0, 3))                  # no momentum either
    assert not np.array_equal(plain.buffer(0, 2), w0[0])
    # layer 2: dW = -decay*B*W (no gradient), W += lr/B * dW (float32 steps)
    B, lr, decay = 8, np.float32(0.01), np.float32(5e-4)
    a1, a2 = np.float32(-decay * np.float32(B)), np.float32(lr / np.float32(B))
    w = w0[2]
    dw = (a1 * w).astype(np.float32)
    want = (w + a2 * dw).astype(np.float32)
    got = stop.buffer(2, 2)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    # the layer above the stop is trained as usual
    assert np.array_equal(stop.buffer(4, 2), plain.buffer(4, 2))
    for n in (plain, stop):
        n.close()


def test_oracle_stopbackward_two_freezes_nothing(oracle):
    """stopbackward=2 on layer 2: the backward loop stops there as for 1
    (NNetwork.c:648 tests nonzero), but only the value 1 freezes the layers
    below (NetworkFactory.c:889-891), so layer 0 keeps train = 1 and takes
    its decay-only update: W += lr/B * (-decay*B*W), no longer its initial
    value, while layer 2's update equals the stopbackward=1 case."""
    one, two = (_tiny_pair(oracle, lambda n, v=v: n.set_layer_options(2, stopbackward=v))[1]
                for v in (1, 2))
    x, t, _ = configs.synthetic_batch("tiny", 3, 8)
    w0 = two.buffer(0, 2).copy()
    one.train(x, t)
    two.train(x, t)
    assert np.array_equal(one.buffer(0, 2), w0)           # frozen by 1
    B, lr, decay = 8, np.float32(0.01), np.float32(5e-4)
    a1, a2 = np.float32(-decay * np.float32(B)), np.float32(lr / np.float32(B))
    want = (w0 + a2 * (a1 * w0).astype(np.float32)).astype(np.float32)
    got = two.buffer(0, 2)
    assert not np.array_equal(got, w0)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    assert np.array_equal(two.buffer(2, 2), one.buffer(2, 2))
    assert np.array_equal(two.buffer(4, 2), one.buffer(4, 2))
    for n in (one, two):
        n.close()


def test_stopbackward_value_kept(tmp_path):
    net = parse(tmp_path, NET + CONV + CONV + "stopbackward=2\n" + TAIL)
    assert net is not None and opts(net, 1)["stopbackward"] == 2
    net.close()


def test_oracle_onlyforward_skips_one_layer(oracle):
    """onlyforward on the max-pool (layer 3): its backward is skipped, so the
    conv layer below gets a zero delta (deltas are zeroed in forward) and
    only its decay / momentum update; the layers above train as usual."""
    plain, skip = _tiny_pair(oracle, lambda n: n.set_layer_options(3, onlyforward=1))
    x, t, _ = configs.synthetic_batch("tiny", 4, 8)
    plain.train(x, t)
    skip.train(x, t)
    assert not np.any(skip.buffer(2, 1))                  # delta of layer 2 stays zero
    assert np.any(plain.buffer(2, 1))
    assert np.array_equal(skip.buffer(4, 2), plain.buffer(4, 2))
    assert not np.any(skip.buffer(2, 7))                  # no scale gradient
    for n in (plain, skip):
        n.close()


def test_oracle_learning_rate_scale_is_a_rate_factor(oracle):
    """learning_rate=2 on layer 0 updates that layer exactly as a global
    learning rate twice as large does (0.01f * 2 == 0.02f); other layers
    keep the base rate."""
    oracle.lib().or_rand_seed(1)
    a = oracle.OracleNet(*configs.dims("tiny", 8))
    configs.build(a, "tiny")
    a.set_layer_options(0, learning_rate_scale=2.0)
    a.finalize()
    oracle.lib().or_rand_seed(1)
    b = oracle.OracleNet(*configs.dims("tiny", 8))
    configs.build(b, "tiny")
    b.hyper(0.02, 0.9, 5e-4)
    b.finalize()
    oracle.lib().or_rand_seed(1)
    c = oracle.OracleNet(*configs.dims("tiny", 8))
    configs.build(c, "tiny")
    c.finalize()
    x, t, _ = configs.synthetic_batch("tiny", 5, 8)
    for n in (a, b, c):
        n.train(x, t)
    assert np.array_equal(a.buffer(0, 2), b.buffer(0, 2))
    assert np.array_equal(a.buffer(2, 2), c.buffer(2, 2))
    assert not np.array_equal(a.buffer(0, 2), c.buffer(0, 2))
    for n in (a, b, c):
        n.close()
