"""Unequal width / height strides (stride_x != stride_y) on the device against
the CPU oracle: the convolution entry points, which run the reference's
per-image im2col / GEMM / col2im passes for such layers
(ConvolutionalLayer.c:337-344, 790-803, 913-945), and the max-pool
(MaxPoolLayer.c:40-41, 237-272, 318-331).  GEMM results within 1e-4
normwise relative error, pool values, indices and sums bit-exact."""
import ctypes as C

import numpy as np
import pytest

import aetcnn
from aetcnn import DeviceArray as D, check
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4
_KEEP = []


@pytest.fixture(autouse=True)
def _keepalive():
    yield
    aetcnn.ops().ach_device_sync()
    _KEEP.clear()


def dev(a):
    d = D.from_numpy(np.ascontiguousarray(a))
    _KEEP.append(d)
    return d


# (B, C, H, W, F, k, stride_x, stride_y, pad)
SHAPES = [
    (2, 3, 9, 8, 4, 3, 2, 1, 1),
    (3, 5, 11, 7, 6, 5, 1, 3, 2),
    (2, 6, 12, 10, 7, 4, 3, 2, 1),
    (2, 4, 7, 9, 5, 1, 1, 2, 0),      # 1x1, stride_x 1 (im2col, not the direct read)
    (4, 16, 20, 24, 40, 3, 2, 1, 1),  # GEMMs past one tile
]


def _inputs(shape, seed):
    B, Cc, H, W, F, k, sx, sy, p = shape
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (B, Cc, H, W)).astype(np.float32)
    w = (rng.standard_normal((F, Cc, k, k)) * 0.1).astype(np.float32)
    OH, OW = (H + 2 * p - k) // sy + 1, (W + 2 * p - k) // sx + 1
    dy = rng.uniform(-1, 1, (B, F, OH, OW)).astype(np.float32)
    return x, w, dy


def _desc(shape):
    B, Cc, H, W, F, k, sx, sy, p = shape
    return aetcnn.ConvDesc(B, Cc, H, W, F, k, sx, p, sy)


def _ws(n):
    return D(max(n, 4) // 4)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv_xy_forward(gpu, oracle, shape):
    B, Cc, H, W, F, k, sx, sy, p = shape
    x, w, _ = _inputs(shape, 1)
    ref = oracle.conv_forward(x, w, F, k, sx, p, stride_y=sy)
    d = _desc(shape)
    assert (gpu.ach_conv_out_h(C.byref(d)), gpu.ach_conv_out_w(C.byref(d))) == ref.shape[2:]
    col = Cc * k * k * ref.shape[2] * ref.shape[3] * 4
    assert gpu.ach_conv_fwd_workspace(C.byref(d)) == col
    dx, dw = dev(x), dev(w)
    ws = _ws(col)
    y = dev(np.full(ref.shape, 7.0, np.float32))  # overwritten
    check(gpu.ach_conv_fwd(C.byref(d), dx.ptr, dw.ptr, y.ptr, ws.ptr, col, None))
    got = y.numpy()
    assert rel_err(got, ref) < TOL
    # the prepared forward reads the k-major filter that
    # ach_conv_prepare_filters makes (no flipped copy for such a layer)
    wt, wft = D((w.size,)), dev(np.full(w.size, 3.0, np.float32))
    job = aetcnn.FilterJob(d, dw.ptr, wt.ptr, wft.ptr)
    check(gpu.ach_conv_prepare_filters(1, C.byref(job), None))
    assert np.array_equal(wt.numpy().reshape(-1), w.reshape(F, -1).T.reshape(-1))
    assert np.all(wft.numpy() == 3.0)
    y2 = D(ref.shape)
    check(gpu.ach_conv_fwd_prepared(C.byref(d), dx.ptr, wt.ptr, y2.ptr, ws.ptr, col, None))
    assert rel_err(y2.numpy(), ref) < TOL
    # bias + activation: the prepared forward, ach_add_bias and ach_activate
    bias = np.random.default_rng(5).uniform(-0.5, 0.5, F).astype(np.float32)
    db = dev(bias)
    for act in (aetcnn.LEAKY, aetcnn.RELU, aetcnn.LINEAR, aetcnn.LOGISTIC):
        y3 = D(ref.shape)
        check(gpu.ach_conv_fwd_bias_act_prepared(C.byref(d), dx.ptr, wt.ptr, db.ptr, act, y3.ptr,
                                                 ws.ptr, col, None))
        y4 = D(ref.shape)
        check(gpu.ach_conv_fwd_prepared(C.byref(d), dx.ptr, wt.ptr, y4.ptr, ws.ptr, col, None))
        check(gpu.ach_add_bias(y4.ptr, db.ptr, B, F, ref.shape[2] * ref.shape[3], None))
        check(gpu.ach_activate(y4.ptr, int(np.prod(ref.shape)), act, None))
        assert np.array_equal(y3.numpy().view(np.uint32), y4.numpy().view(np.uint32)), act
    # too small a workspace is refused
    assert gpu.ach_conv_fwd(C.byref(d), dx.ptr, dw.ptr, y.ptr, ws.ptr, col - 4, None) == \
        aetcnn.ACH_EWORKSPACE


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv_xy_backward(gpu, oracle, shape):
    B, Cc, H, W, F, k, sx, sy, p = shape
    x, w, dy = _inputs(shape, 2)
    dw0 = (np.random.default_rng(9).standard_normal(w.shape) * 0.1).astype(np.float32)
    ref_dw, ref_dx = oracle.conv_backward(x, dy, w, k, sx, p, dw0=dw0, stride_y=sy)
    d = _desc(shape)
    col = Cc * k * k * dy.shape[2] * dy.shape[3] * 4
    assert gpu.ach_conv_bwd_data_workspace(C.byref(d)) == col
    assert gpu.ach_conv_bwd_filter_workspace(C.byref(d)) == col
    assert gpu.ach_conv_bwd_data_reads_w(C.byref(d)) == 1
    ws = _ws(col)
    dx_, ddy, dwt = dev(x), dev(dy), dev(w)
    ddx = dev(np.full(x.shape, 5.0, np.float32))  # overwritten
    check(gpu.ach_conv_bwd_data(C.byref(d), ddy.ptr, dwt.ptr, ddx.ptr, ws.ptr, col, None))
    assert rel_err(ddx.numpy(), ref_dx) < TOL
    # no prepared input gradient for such a layer
    assert gpu.ach_conv_bwd_data_prepared(C.byref(d), ddy.ptr, dwt.ptr, dwt.ptr, ddx.ptr, ws.ptr,
                                          col, None) == aetcnn.ACH_EUNSUPPORTED
    ddw = dev(dw0)
    check(gpu.ach_conv_bwd_filter(C.byref(d), dx_.ptr, ddy.ptr, ddw.ptr, ws.ptr, col, None))
    assert rel_err(ddw.numpy(), ref_dw) < TOL
    # with the SGD step: the weight gradient, then ach_sgd_update, bit for bit
    dc, lc, mom = np.float32(-5e-4 * B), np.float32(0.01 / B), np.float32(0.9)
    wa, dwa, wb, dwb = dev(w), dev(dw0), dev(w), dev(dw0)
    check(gpu.ach_conv_bwd_filter(C.byref(d), dx_.ptr, ddy.ptr, dwa.ptr, ws.ptr, col, None))
    check(gpu.ach_sgd_update(w.size, wa.ptr, dwa.ptr, dc, lc, mom, None))
    check(gpu.ach_conv_bwd_filter_sgd(C.byref(d), dx_.ptr, ddy.ptr, wb.ptr, dwb.ptr, dc, lc, mom,
                                      ws.ptr, col, None))
    assert np.array_equal(wa.numpy().view(np.uint32), wb.numpy().view(np.uint32))
    assert np.array_equal(dwa.numpy().view(np.uint32), dwb.numpy().view(np.uint32))


def test_conv_xy_fully_connected_geometry(gpu, oracle):
    """A kernel covering the whole unpadded input has one output position
    whatever the strides: it keeps the fully connected path (no copy of the
    filter, no column buffer) and matches the square-stride layer."""
    shape = (8, 16, 3, 3, 20, 3, 2, 1, 0)
    B, Cc, H, W, F, k, sx, sy, p = shape
    x, w, dy = _inputs(shape, 3)
    d, sq = _desc(shape), aetcnn.ConvDesc(B, Cc, H, W, F, k, 1, p)
    assert gpu.ach_conv_is_fully_connected(C.byref(d)) == 1
    assert gpu.ach_conv_fwd_workspace(C.byref(d)) == gpu.ach_conv_fwd_workspace(C.byref(sq))
    ref = oracle.conv_forward(x, w, F, k, sx, p, stride_y=sy)
    ws_n = gpu.ach_conv_fwd_workspace(C.byref(d))
    ws = _ws(ws_n)
    dx, dw, y = dev(x), dev(w), D(ref.shape)
    check(gpu.ach_conv_fwd_prepared(C.byref(d), dx.ptr, dw.ptr, y.ptr, ws.ptr, ws_n, None))
    assert rel_err(y.numpy(), ref) < TOL


# (B, C, H, W, size, stride_x, stride_y, padding)
POOLS = [
    (2, 3, 9, 11, 2, 2, 1, 1),
    (2, 2, 16, 16, 2, 1, 2, 1),
    (3, 2, 13, 10, 3, 2, 3, 2),
    (1, 4, 20, 7, 3, 3, 1, 0),
    (2, 3, 150, 40, 2, 1, 2, 1),      # large planes
]


@pytest.mark.parametrize("B,Cc,H,W,size,sx,sy,pad", POOLS)
def test_maxpool_xy_bit_exact(gpu, oracle, B, Cc, H, W, size, sx, sy, pad):
    rng = np.random.default_rng(H * W + size + sx)
    x = rng.integers(-3, 4, (B, Cc, H, W)).astype(np.float32)  # ties: first max wins
    out, idx = oracle.maxpool_forward(x, size, sx, pad, stride_y=sy)
    assert out.shape[2:] == ((H + pad - size) // sy + 1, (W + pad - size) // sx + 1)
    dx, dout, didx = dev(x), D(out.shape), D(out.shape, np.int32)
    check(gpu.ach_maxpool_fwd_xy(dx.ptr, B, Cc, H, W, size, sx, sy, pad, dout.ptr, didx.ptr,
                                 None))
    assert np.array_equal(dout.numpy(), out)
    assert np.array_equal(didx.numpy(), idx)
    g = rng.standard_normal(out.shape).astype(np.float32)
    g.reshape(-1)[::7] = -0.0
    din0 = rng.standard_normal(x.shape).astype(np.float32)
    ref = oracle.maxpool_backward(g, idx, din0)
    ddin, dg = dev(din0), dev(g)
    check(gpu.ach_maxpool_bwd_xy(dg.ptr, didx.ptr, B, Cc, H, W, size, sx, sy, pad, ddin.ptr, 1,
                                 None))
    assert np.array_equal(ddin.numpy(), ref)
    ref0 = oracle.maxpool_backward(g, idx, np.zeros_like(x))
    ddin0 = dev(np.full(x.shape, np.nan, np.float32))
    check(gpu.ach_maxpool_bwd_xy(dg.ptr, didx.ptr, B, Cc, H, W, size, sx, sy, pad, ddin0.ptr, 0,
                                 None))
    assert np.array_equal(ddin0.numpy().view(np.uint32), ref0.view(np.uint32))


def test_maxpool_xy_equal_strides_and_errors(gpu, oracle):
    """Equal strides take the square-stride kernels (the same results); bad
    strides are refused before any launch."""
    rng = np.random.default_rng(4)
    x = rng.integers(-3, 4, (2, 3, 12, 12)).astype(np.float32)
    out, idx = oracle.maxpool_forward(x, 2, 2, 1)
    dx, dout, didx = dev(x), D(out.shape), D(out.shape, np.int32)
    check(gpu.ach_maxpool_fwd_xy(dx.ptr, 2, 3, 12, 12, 2, 2, 2, 1, dout.ptr, didx.ptr, None))
    assert np.array_equal(dout.numpy(), out) and np.array_equal(didx.numpy(), idx)
    for sx, sy in ((0, 2), (2, 0), (-1, 1)):
        assert gpu.ach_maxpool_fwd_xy(dx.ptr, 2, 3, 12, 12, 2, sx, sy, 1, dout.ptr, didx.ptr,
                                      None) == aetcnn.ACH_EINVAL
        assert gpu.ach_maxpool_bwd_xy(dout.ptr, didx.ptr, 2, 3, 12, 12, 2, sx, sy, 1, dx.ptr, 0,
                                      None) == aetcnn.ACH_EINVAL


STRIDENET_CFG = """[net]
batch=16
height=16
width=32
channels=3
learning_rate=0.05
momentum=0.9
decay=0.0005

[convolutional]
batch_normalize=1
filters=8
size=3
stride_x=2
stride_y=1
pad=1
activation=leaky

[maxpool]
size=2
stride_x=1
stride_y=2
padding=1

[convolutional]
filters=12
size=3
stride=1
pad=1
activation=relu

[maxpool]
size=2
stride=2
stride_y=1
padding=0

[convolutional]
filters=16
size=3
stride=1
stride_y=2
pad=1
activation=leaky

[convolutional]
filters=10
size=1
stride_x=2
stride_y=1
activation=linear

[avgpool]
[softmax]
"""


def test_cfg_unequal_strides_drive_same_network(gpu, tmp_path):
    """stride_x / stride_y keys (NetworkFactory.c:83-90, 544-547) build the
    network of the builder calls with the same strides: identical layer
    shapes, and two training steps with identical losses."""
    from aetcnn import configs
    cfg = tmp_path / "xy.cfg"
    cfg.write_text(STRIDENET_CFG)
    aetcnn.net_lib().an_rand_seed(1)
    a = aetcnn.Network.from_cfg(str(cfg))
    aetcnn.net_lib().an_rand_seed(1)
    B, h, w, c = configs.dims("stridenet")
    b = aetcnn.Network(B, h, w, c)
    configs.build(b, "stridenet")
    b.finalize()
    assert a.n_layers() == b.n_layers()
    for i in range(a.n_layers()):
        assert a.shape(i) == b.shape(i), i
    x, truth, _ = configs.synthetic_batch("stridenet", 3)
    for _ in range(2):
        assert a.train(x, truth) == b.train(x, truth)
    a.close()
    b.close()
