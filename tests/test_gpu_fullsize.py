"""Parity at the benchmark sizes: config 1 (the conv sweep at batch 128) and
config 2 (the HBM-bound operators on [512][128][32][32]) on the very arrays
bench.py times (bench.config1_inputs / bench.config2_inputs), against the
CPU oracle, and for the batch-norm statistics also against float64 closed
forms.

Bars as in test_gpu_ops.py: argmax indices and element-wise ops with the
same arithmetic bit-exact; reductions and GEMMs within 1e-4 normwise
relative.  Per-channel reductions over 524,288 elements are where the
reference's own sequential fp32 sums (NormData.c:141-186, DeltaData.c:23-58,
ScaleData.c:76-107) drift furthest from exact arithmetic: there the GPU must
be within 1e-5 of float64 and no further from the oracle than the oracle is
from float64 (plus 1e-5)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import aetcnn
from aetcnn import DeviceArray as D, check
from conftest import ROOT, rel_err
from refs64 import bn_backward_ref

sys.path.insert(0, ROOT)
import bench  # noqa: E402  (the benchmark's input generators)

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def c2(gpu):
    return bench.config2_inputs()


def _reduction_ok(name, got, ref, exact):
    """got (GPU) vs ref (oracle), both judged against float64 `exact`."""
    e = rel_err(got, ref)
    if e < TOL:
        return
    e_gpu, e_ref = rel_err(got, exact), rel_err(ref, exact)
    assert e_gpu < 1e-5 and e <= e_ref + 1e-5, (name, e, e_gpu, e_ref)


def test_config2_batchnorm(gpu, oracle, c2):
    """BN training forward (statistics, rolling .9/.1, normalize) and
    backward (scale gradient, mean / variance deltas, delta) at full size,
    with the scales / biases / statistics bench.py starts from."""
    B, Cc, H, W = bench.BW_SHAPE
    HW = H * W
    x = c2["x"]
    ones, zeros = np.ones(Cc, np.float32), np.zeros(Cc, np.float32)
    f = oracle.bn_forward(x.reshape(B, Cc, H, W), ones, zeros, zeros, zeros)
    dx, dout = D.from_numpy(x), D(x.size)
    dsc, dbi = D.from_numpy(ones), D.from_numpy(zeros)
    dm, dv, drm, drv = D(Cc), D(Cc), D.from_numpy(zeros), D.from_numpy(zeros)
    ws = gpu.ach_bn_workspace(B, Cc, HW)
    dws = D(ws // 4 + 64)
    check(gpu.ach_bn_train_fwd_from_x(dx.ptr, dout.ptr, B, Cc, HW, dsc.ptr, dbi.ptr, dm.ptr,
                                      dv.ptr, drm.ptr, drv.ptr, aetcnn.LINEAR, dws.ptr, ws, None))
    xr = x.reshape(B, Cc, HW)
    n = B * HW
    mean64 = xr.sum(axis=(0, 2), dtype=np.float64) / n
    var64 = ((xr - mean64[None, :, None].astype(np.float32)).astype(np.float64) ** 2).sum(
        axis=(0, 2)) / (n - 1)
    mean, var = dm.numpy(), dv.numpy()
    assert rel_err(mean, mean64) < 1e-5 and rel_err(var, var64) < 1e-5
    _reduction_ok("mean", mean, f["mean"], mean64)
    _reduction_ok("variance", var, f["var"], var64)
    assert rel_err(drm.numpy(), f["rm"]) < 1e-5 and rel_err(drv.numpy(), f["rv"]) < 1e-5
    assert rel_err(dout.numpy(), f["out"]) < TOL
    assert np.array_equal(dx.numpy(), x)
    del dout
    # backward on the oracle's statistics (teacher-forced), x_norm recomputed
    dm.upload(f["mean"])
    dv.upload(f["var"])
    delta = c2["delta"]
    ref = oracle.bn_backward(delta.reshape(B, Cc, H, W), f["x"], f["xn"], f["mean"], f["var"],
                             ones, zeros)
    ddelta, dsu, dmd, dvd = D.from_numpy(delta), D.from_numpy(zeros), D(Cc), D(Cc)
    check(gpu.ach_bn_bwd(ddelta.ptr, B, Cc, HW, dx.ptr, None, dm.ptr, dv.ptr, dsc.ptr, dbi.ptr,
                         dsu.ptr, dmd.ptr, dvd.ptr, aetcnn.LINEAR, dws.ptr, ws, None))
    got = ddelta.numpy()
    assert rel_err(got, ref["delta"]) < TOL
    out64, dgamma64 = bn_backward_ref(delta.reshape(B, Cc, H, W), None,
                                      x.reshape(B, Cc, H, W), f["mean"], f["var"], ones,
                                      act_leaky=False)
    assert rel_err(got, out64) < TOL
    _reduction_ok("scale_updates", dsu.numpy(), ref["scale_updates"], dgamma64)
    d64 = delta.reshape(B, Cc, HW).astype(np.float64)
    xc64 = xr.astype(np.float64) - f["mean"].astype(np.float64)[None, :, None]
    v64 = f["var"].astype(np.float64)
    md64 = -d64.sum(axis=(0, 2)) / np.sqrt(v64 + 1e-5)
    vd64 = (d64 * xc64).sum(axis=(0, 2)) * -0.5 * (v64 + 1e-5) ** -1.5
    _reduction_ok("mean_delta", dmd.numpy(), ref["mean_delta"], md64)
    _reduction_ok("variance_delta", dvd.numpy(), ref["var_delta"], vd64)


def test_config2_leaky(gpu, oracle, c2):
    """leaky(0.1) forward and gradient over 67 M elements, bit-exact."""
    x, delta = c2["x"], c2["delta"]
    d = D.from_numpy(x)
    check(gpu.ach_activate(d.ptr, x.size, aetcnn.LEAKY, None))
    y = d.numpy()
    assert np.array_equal(y.view(np.uint32), oracle.activate(x, aetcnn.LEAKY).view(np.uint32))
    dd = D.from_numpy(delta)
    check(gpu.ach_gradient(d.ptr, x.size, aetcnn.LEAKY, dd.ptr, None))
    ref = oracle.gradient(y, aetcnn.LEAKY, delta)
    assert np.array_equal(dd.numpy().view(np.uint32), ref.view(np.uint32))


def test_config2_maxpool(gpu, oracle, c2):
    """2x2/2 max-pool (darknet padding 1) forward with int32 global argmax
    indices and backward (delta_in written, accumulate = 0), bit-exact."""
    B, Cc, H, W = bench.BW_SHAPE
    x = c2["x"].reshape(B, Cc, H, W)
    out, idx = oracle.maxpool_forward(x, 2, 2, 1)
    dx, dout, didx = D.from_numpy(x), D(out.shape), D(out.shape, np.int32)
    check(gpu.ach_maxpool_fwd(dx.ptr, B, Cc, H, W, 2, 2, 1, dout.ptr, didx.ptr, None))
    assert np.array_equal(didx.numpy(), idx)
    assert np.array_equal(dout.numpy().view(np.uint32), out.view(np.uint32))
    g = c2["pool_delta"].reshape(out.shape)
    ref = oracle.maxpool_backward(g, idx, np.zeros_like(x))
    dg = D.from_numpy(g)
    check(gpu.ach_maxpool_bwd(dg.ptr, didx.ptr, B, Cc, H, W, 2, 2, 1, dx.ptr, 0, None))
    assert np.array_equal(dx.numpy().view(np.uint32), ref.view(np.uint32))


def test_config2_sgd(gpu, oracle, c2):
    """SGD momentum + decay over the 60 M-parameter flat buffer, against the
    oracle's ConvolutionalLayer.update (both contract to FMA; at most 1 ulp
    apart)."""
    lr, mom, decay, batch = bench.SGD_HYPER
    w, v = c2["sgd_w"], c2["sgd_v"]
    e = np.zeros(0, np.float32)
    rw, rv, _, _, _, _ = oracle.conv_update(w, v, e, e, None, None, batch, lr, mom, decay)
    dw, dv = D.from_numpy(w), D.from_numpy(v)
    check(gpu.ach_sgd_update(w.size, dw.ptr, dv.ptr, -decay * batch, lr / batch, mom, None))
    for got, ref in ((dw.numpy(), rw), (dv.numpy(), rv)):
        ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert ulp.max() <= 1 and rel_err(got, ref) < 1e-7


@pytest.mark.parametrize("shape", bench.SWEEP, ids=lambda s: "%d-%d@%d-k%d" % s[:4])
def test_config1_sweep_b128(gpu, oracle, shape):
    """Each config-1 layer at batch 128: forward, input gradient (the
    3-channel first layer's too) and weight gradient against the oracle."""
    ci, co, hw, k, p = shape
    B = 128
    x, w, dy = bench.config1_inputs(np.random.default_rng(ci * 1000 + co), B, ci, co, hw, k, p)
    d = aetcnn.ConvDesc(B, ci, hw, hw, co, k, 1, p)
    ws = max(gpu.ach_conv_fwd_workspace(C.byref(d)), gpu.ach_conv_bwd_data_workspace(C.byref(d)),
             gpu.ach_conv_bwd_filter_workspace(C.byref(d)), 256)
    dws = D(ws // 4)
    dx, dwt, ddy = D.from_numpy(x), D.from_numpy(w), D.from_numpy(dy)
    y = D(dy.shape)
    check(gpu.ach_conv_fwd(C.byref(d), dx.ptr, dwt.ptr, y.ptr, dws.ptr, ws, None))
    ref_y = oracle.conv_forward(x, w, co, k, 1, p)
    assert rel_err(y.numpy(), ref_y) < TOL
    ref_dw, ref_dx = oracle.conv_backward(x, dy, w, k, 1, p)
    gx = D(x.shape)
    check(gpu.ach_conv_bwd_data(C.byref(d), ddy.ptr, dwt.ptr, gx.ptr, dws.ptr, ws, None))
    assert rel_err(gx.numpy(), ref_dx) < TOL
    gw = D(w.shape)
    gw.zero()
    check(gpu.ach_conv_bwd_filter(C.byref(d), dx.ptr, ddy.ptr, gw.ptr, dws.ptr, ws, None))
    assert rel_err(gw.numpy(), ref_dw) < TOL
