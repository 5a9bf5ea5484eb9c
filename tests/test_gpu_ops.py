"""Per-operator parity: HIP kernels (through the C-ABI of libach.so) against
the CPU oracle on identical seeded inputs.

Bars: integer outputs (argmax indices, dropout masks, im2col copies) and
elementwise ops with identical arithmetic are bit-exact; reductions and GEMMs
are within 1e-4 normwise relative error (the tolerance the reference's own
GPU-vs-CPU compare blocks use, DnnUtils.c:377-392)."""
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
    """Device arrays made by dev() live until the test ends, so a pointer
    taken from a temporary (dev(x).ptr) is never freed before its kernel runs."""
    yield
    aetcnn.ops().ach_device_sync()
    _KEEP.clear()


def dev(a):
    d = D.from_numpy(np.ascontiguousarray(a))
    _KEEP.append(d)
    return d


def conv_desc(B, Cc, H, W, F, k, s, p):
    return aetcnn.ConvDesc(B, Cc, H, W, F, k, s, p)


# ---------------------------------------------------------------------------
@pytest.mark.parametrize("TA,TB", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(67, 45, 33), (256, 300, 129), (10, 128, 512), (1, 1, 1)])
def test_gemm(gpu, oracle, TA, TB, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 3 + K + TA * 2 + TB)
    A = rng.standard_normal((K, M) if TA else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if TB else (K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    lda, ldb = A.shape[1], B.shape[1]
    for alpha, beta in [(1.0, 1.0), (0.5, 0.0), (1.0, 0.25)]:
        ref = oracle.gemm(TA, TB, M, N, K, alpha, A, lda, B, ldb, beta, C0, N)
        dA, dB, dC = dev(A), dev(B), dev(C0)
        check(gpu.ach_gemm(TA, TB, M, N, K, alpha, dA.ptr, lda, dB.ptr, ldb, beta, dC.ptr, N, None))
        got = dC.numpy()
        assert rel_err(got, ref) < 1e-5, (alpha, beta)


@pytest.mark.parametrize("Cc,H,W,k,p,s,dl", [(3, 7, 9, 3, 1, 1, 1), (4, 12, 12, 5, 2, 2, 1),
                                             (2, 35, 35, 11, 0, 4, 1), (6, 6, 6, 6, 0, 1, 1),
                                             (5, 8, 8, 1, 0, 1, 1),
                                             (3, 11, 9, 3, 2, 1, 2),   # dilated (Im2Col.c ext)
                                             (2, 13, 13, 3, 3, 2, 3)])
def test_im2col_col2im_bit_exact(gpu, oracle, Cc, H, W, k, p, s, dl):
    rng = np.random.default_rng(Cc * H + k)
    im = rng.standard_normal((Cc, H, W)).astype(np.float32)
    ek = dl * (k - 1) + 1
    OH, OW = (H + 2 * p - ek) // s + 1, (W + 2 * p - ek) // s + 1
    col_ref = np.zeros(Cc * k * k * OH * OW, np.float32)
    oracle.lib().or_im2col(oracle.P(im), Cc, H, W, k, k, p, p, s, s, dl, dl, oracle.P(col_ref))
    dim, dcol = dev(im), D(col_ref.shape)
    check(gpu.ach_im2col(dim.ptr, Cc, H, W, k, k, p, p, s, s, dl, dl, dcol.ptr, None))
    assert np.array_equal(dcol.numpy(), col_ref)
    col = rng.standard_normal(col_ref.shape).astype(np.float32)
    im_ref = np.zeros_like(im)
    oracle.lib().or_col2im(oracle.P(col), Cc, H, W, k, k, p, p, s, s, dl, dl, oracle.P(im_ref))
    dcol2, dim2 = dev(col), dev(np.full_like(im, 7.0))  # col2im must overwrite
    check(gpu.ach_col2im(dcol2.ptr, Cc, H, W, k, k, p, p, s, s, dl, dl, dim2.ptr, None))
    assert np.array_equal(dim2.numpy(), im_ref)


CONV_SHAPES = [
    # (B, C, H, W, F, k, s, p)
    (2, 3, 32, 32, 128, 3, 1, 1),
    (2, 128, 32, 32, 128, 3, 1, 1),
    (2, 128, 16, 16, 256, 3, 1, 1),
    (2, 256, 16, 16, 256, 3, 1, 1),
    (2, 256, 8, 8, 512, 3, 1, 1),
    (2, 512, 8, 8, 512, 3, 1, 1),
    (2, 512, 8, 8, 10, 1, 1, 0),
    (3, 5, 9, 7, 10, 3, 1, 1),
    (2, 16, 13, 13, 24, 5, 1, 2),
    (2, 3, 35, 35, 8, 11, 4, 0),
    (4, 32, 6, 6, 40, 6, 1, 0),
    (5, 7, 1, 1, 9, 1, 1, 0),
    (3, 6, 12, 12, 20, 3, 1, 1),   # vector im2col loader, partial N tile, ragged K
    (2, 8, 10, 10, 16, 3, 1, 0),   # vector loader without padding (dgrad: pad 2)
    (2, 4, 4, 4, 8, 3, 1, 1),      # narrowest input the vector loader takes
    # weight gradient in the chunked K order (OH*OW % 16 == 0):
    (9, 16, 8, 8, 32, 3, 1, 1),    # odd batch split into uneven image ranges
    (4, 8, 16, 16, 16, 3, 2, 1),   # stride 2
    (4, 6, 8, 8, 12, 5, 1, 2),     # 5x5
    (2, 96, 9, 9, 80, 5, 1, 2),    # 5x5 with 80 / 96 filters: 96-row tiles
    (6, 24, 4, 4, 20, 1, 1, 0),    # 1x1 on a 16-position plane
    # 96-row tiles with the generic loader (65-96 filters / input channels):
    (2, 3, 35, 35, 96, 11, 4, 0),  # AlexNet conv1 shape class
    (2, 80, 9, 9, 72, 7, 1, 3),    # 7x7: forward M=72, input gradient M=80
    (2, 16, 8, 8, 80, 3, 1, 1),    # weight gradient 96 x 128 tiles, chunked K, 3x3
    (3, 4, 11, 11, 96, 4, 1, 0),   # weight gradient 96 x 128 tiles, chunked K, 4x4
    (8, 16, 5, 5, 24, 3, 1, 1),    # 25 positions: the (image, position) order
    # shallow im2col (C*k*k <= 32: the whole K in MFMA registers, no LDS):
    (3, 2, 9, 11, 40, 3, 2, 1),    # stride 2, 33-64 filters
    (2, 1, 12, 10, 70, 5, 1, 2),   # 5x5 (kernel size at run time), ragged M
    (3, 3, 7, 5, 16, 3, 1, 0),     # no padding, 45 output columns
    (2, 32, 5, 5, 33, 1, 1, 0),    # K = 32 exactly, 33 filters
    # fully connected layers (1x1 of a 1x1 input, after flattening):
    (16, 256, 3, 3, 200, 3, 1, 0), # kernel covering a 3x3 input: 2304 -> 200
    (8, 64, 1, 1, 48, 1, 1, 0),    # 64 -> 48, 64-row tiles
    (16, 2048, 1, 1, 8192, 1, 1, 0),  # pairs of K slices per workgroup (fwd and dgrad)
    (4, 1000, 1, 1, 256, 1, 1, 0),  # 128-row tiles, K ending inside a 32-wide k-tile
    (3, 1001, 1, 1, 130, 1, 1, 0),  # K and M not multiples of 4: scalar loaders
    # split K on 169-position planes with N % 4 == 0: partials reduced in
    # their own order, four sums of one plane stored at once
    (4, 64, 13, 13, 96, 3, 1, 1),
    # 11x11 without padding: k-tiles of two filter rows (row-tap loaders)
    (2, 4, 23, 23, 64, 11, 2, 0),  # 44 filter rows: 22 pairs
    (3, 5, 21, 21, 12, 11, 1, 0),  # 55 rows: the last pair half empty
    # one-pass 1x1 weight gradient (at most 16 filters, planes of <= 256):
    (3, 37, 7, 9, 16, 1, 1, 0),    # channels not a multiple of 4, odd plane
    (2, 5, 16, 16, 1, 1, 1, 0),    # one filter, a 256-position plane
    # 3x3 forwards with an odd k-tile count (C/2 = 17): the K split gives
    # slices of 9 and 8 tiles, which must not share one workgroup
    (2, 34, 8, 8, 128, 3, 1, 1),   # one tile split in two
    (16, 34, 32, 32, 512, 3, 1, 1),  # 512 tiles
]


def _conv_inputs(shape, seed):
    B, Cc, H, W, F, k, s, p = shape
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (B, Cc, H, W)).astype(np.float32)
    w = (rng.standard_normal((F, Cc, k, k)) * 0.05).astype(np.float32)
    OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    dy = rng.uniform(-1, 1, (B, F, OH, OW)).astype(np.float32)
    return x, w, dy


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv_fwd(gpu, oracle, shape):
    B, Cc, H, W, F, k, s, p = shape
    x, w, _ = _conv_inputs(shape, 1)
    ref = oracle.conv_forward(x, w, F, k, s, p)
    d = conv_desc(*shape)
    dx, dw, dy = dev(x), dev(w), D(ref.shape)
    check(gpu.ach_fill(dy.ptr, ref.size, 123.0, None))  # must be overwritten
    ws = gpu.ach_conv_fwd_workspace(C.byref(d))
    dws = D(max(ws, 4) // 4)
    check(gpu.ach_conv_fwd(C.byref(d), dx.ptr, dw.ptr, dy.ptr, dws.ptr, ws, None))
    assert rel_err(dy.numpy(), ref) < TOL


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv_bwd_data(gpu, oracle, shape):
    B, Cc, H, W, F, k, s, p = shape
    x, w, dy = _conv_inputs(shape, 2)
    _, ref = oracle.conv_backward(x, dy, w, k, s, p)
    d = conv_desc(*shape)
    ddy, dw, ddx = dev(dy), dev(w), dev(np.full(x.shape, 5.0, np.float32))
    ws = gpu.ach_conv_bwd_data_workspace(C.byref(d))
    dws = D(max(ws, 4) // 4)
    check(gpu.ach_conv_bwd_data(C.byref(d), ddy.ptr, dw.ptr, ddx.ptr, dws.ptr, ws, None))
    assert rel_err(ddx.numpy(), ref) < TOL


@pytest.mark.parametrize("shape", CONV_SHAPES + [(2, 3, 227, 227, 96, 11, 4, 0)],
                         ids=lambda s: "x".join(map(str, s)))
def test_conv_bwd_filter_sgd(gpu, shape):
    """ach_conv_bwd_filter_sgd == ach_conv_bwd_filter + ach_sgd_update over
    the weights, bit for bit, whether the update runs in the unsplit GEMM's
    epilogue, the split-K reduction (one or two levels) or a pass of its own
    (ConvolutionalLayer.c:913-929, 959-980)."""
    B, Cc, H, W, F, k, s, p = shape
    x, w, dy = _conv_inputs(shape, 41)
    rng = np.random.default_rng(42)
    dw0 = (rng.standard_normal(w.shape) * 0.1).astype(np.float32)
    d = conv_desc(*shape)
    ws = gpu.ach_conv_bwd_filter_workspace(C.byref(d))
    dws = D(max(ws, 4) // 4)
    dc, lc, mom = np.float32(-5e-4 * B), np.float32(0.01 / B), np.float32(0.9)
    dx_, ddy = dev(x), dev(dy)
    wa, dwa, wb, dwb = dev(w), dev(dw0), dev(w), dev(dw0)
    check(gpu.ach_conv_bwd_filter(C.byref(d), dx_.ptr, ddy.ptr, dwa.ptr, dws.ptr, ws, None))
    check(gpu.ach_sgd_update(w.size, wa.ptr, dwa.ptr, dc, lc, mom, None))
    check(gpu.ach_conv_bwd_filter_sgd(C.byref(d), dx_.ptr, ddy.ptr, wb.ptr, dwb.ptr, dc, lc, mom,
                                      dws.ptr, ws, None))
    assert np.array_equal(wa.numpy().view(np.uint32), wb.numpy().view(np.uint32)), shape
    assert np.array_equal(dwa.numpy().view(np.uint32), dwb.numpy().view(np.uint32)), shape


@pytest.mark.parametrize("shape", CONV_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_conv_bwd_filter(gpu, oracle, shape):
    B, Cc, H, W, F, k, s, p = shape
    x, w, dy = _conv_inputs(shape, 3)
    dw0 = (np.random.default_rng(9).standard_normal(w.shape) * 0.1).astype(np.float32)
    ref, _ = oracle.conv_backward(x, dy, w, k, s, p, dw0=dw0, want_dx=False)
    d = conv_desc(*shape)
    dx, ddy, ddw = dev(x), dev(dy), dev(dw0)
    ws = gpu.ach_conv_bwd_filter_workspace(C.byref(d))
    dws = D(max(ws, 4) // 4)
    check(gpu.ach_conv_bwd_filter(C.byref(d), dx.ptr, ddy.ptr, ddw.ptr, dws.ptr, ws, None))
    assert rel_err(ddw.numpy(), ref) < TOL


def test_conv_bwd_filter_full_batch_split_k(gpu, oracle):
    """B=16 forces split-K with several partials; compare to the oracle."""
    shape = (16, 64, 16, 16, 64, 3, 1, 1)
    B, Cc, H, W, F, k, s, p = shape
    x, w, dy = _conv_inputs(shape, 4)
    ref, _ = oracle.conv_backward(x, dy, w, k, s, p, want_dx=False)
    d = conv_desc(*shape)
    assert gpu.ach_conv_bwd_filter_workspace(C.byref(d)) > 0
    dx, ddy, ddw = dev(x), dev(dy), dev(np.zeros_like(w))
    ws = gpu.ach_conv_bwd_filter_workspace(C.byref(d))
    dws = D(ws // 4)
    check(gpu.ach_conv_bwd_filter(C.byref(d), dx.ptr, ddy.ptr, ddw.ptr, dws.ptr, ws, None))
    got = ddw.numpy()
    assert rel_err(got, ref) < TOL
    # deterministic: a second run from zero gives identical bits
    ddw.zero()
    check(gpu.ach_conv_bwd_filter(C.byref(d), dx.ptr, ddy.ptr, ddw.ptr, dws.ptr, ws, None))
    assert np.array_equal(ddw.numpy(), got)


def test_conv_workspace_errors(gpu):
    d = conv_desc(16, 64, 16, 16, 64, 3, 1, 1)
    x, dy, dw = D((16, 64, 16, 16)), D((16, 64, 16, 16)), D((64, 64, 3, 3))
    assert gpu.ach_conv_bwd_filter(C.byref(d), x.ptr, dy.ptr, dw.ptr, None, 0, None) == \
        aetcnn.ACH_EWORKSPACE
    bad = conv_desc(0, 64, 16, 16, 64, 3, 1, 1)
    assert gpu.ach_conv_fwd(C.byref(bad), x.ptr, dw.ptr, dy.ptr, None, 0, None) == aetcnn.ACH_EINVAL


# ---------------------------------------------------------------------------
def _bn_inputs(B, Cc, H, W, seed):
    rng = np.random.default_rng(seed)
    out = (rng.standard_normal((B, Cc, H, W)) * 1.3 + 0.2).astype(np.float32)
    scales = rng.uniform(0.5, 1.5, Cc).astype(np.float32)
    biases = rng.uniform(-0.2, 0.2, Cc).astype(np.float32)
    rm = rng.uniform(-0.1, 0.1, Cc).astype(np.float32)
    rv = rng.uniform(0.5, 1.5, Cc).astype(np.float32)
    return out, scales, biases, rm, rv


@pytest.mark.parametrize("B,Cc,H,W", [(8, 16, 32, 32), (4, 24, 13, 13), (128, 32, 8, 8),
                                      (3, 5, 1, 1),
                                      # one workgroup per channel (at most 32768 values):
                                      (32, 256, 16, 16), (7, 130, 6, 6), (9, 128, 2, 2)])
@pytest.mark.parametrize("act", [aetcnn.LINEAR, aetcnn.LEAKY])
def test_bn_train_fwd(gpu, oracle, B, Cc, H, W, act):
    out, sc, bi, rm, rv = _bn_inputs(B, Cc, H, W, B + Cc + act)
    ref = oracle.bn_forward(out, sc, bi, rm, rv)
    ref_out = oracle.activate(ref["out"], act)
    d_out, d_x, d_xn = dev(out), D(out.shape), D(out.shape)
    d_sc, d_bi, d_m, d_v, d_rm, d_rv = dev(sc), dev(bi), D(Cc), D(Cc), dev(rm), dev(rv)
    ws = gpu.ach_bn_workspace(B, Cc, H * W)
    d_ws = D(ws // 4 + 1)
    check(gpu.ach_bn_train_fwd(d_out.ptr, B, Cc, H * W, d_sc.ptr, d_bi.ptr, d_m.ptr, d_v.ptr,
                               d_rm.ptr, d_rv.ptr, d_x.ptr, d_xn.ptr, act, d_ws.ptr, ws, None))
    assert np.array_equal(d_x.numpy(), out)
    assert rel_err(d_m.numpy(), ref["mean"]) < 1e-5
    assert rel_err(d_v.numpy(), ref["var"]) < 1e-5
    assert rel_err(d_rm.numpy(), ref["rm"]) < 1e-5
    assert rel_err(d_rv.numpy(), ref["rv"]) < 1e-5
    assert rel_err(d_xn.numpy(), ref["xn"]) < TOL
    assert rel_err(d_out.numpy(), ref_out) < TOL
    # from_x variant writes only out
    d_out2 = D(out.shape)
    d_rm2, d_rv2 = dev(rm), dev(rv)
    check(gpu.ach_bn_train_fwd_from_x(d_x.ptr, d_out2.ptr, B, Cc, H * W, d_sc.ptr, d_bi.ptr,
                                      d_m.ptr, d_v.ptr, d_rm2.ptr, d_rv2.ptr, act, d_ws.ptr, ws,
                                      None))
    assert np.array_equal(d_out2.numpy(), d_out.numpy())


@pytest.mark.parametrize("B,Cc,H,W", [(8, 16, 32, 32), (4, 24, 13, 13), (3, 5, 1, 1)])
@pytest.mark.parametrize("act", [aetcnn.LINEAR, aetcnn.LEAKY, aetcnn.RELU])
def test_bn_infer(gpu, oracle, B, Cc, H, W, act):
    """ach_bn_infer vs NormData.normalizeByRoll + activation; in place too."""
    out, sc, bi, rm, rv = _bn_inputs(B, Cc, H, W, 3 * B + Cc + act)
    ref = oracle.activate(oracle.bn_normalize_roll(out, rm, rv, sc, bi), act)
    d_x, d_out = dev(out), D(out.shape)
    d_sc, d_bi, d_rm, d_rv = dev(sc), dev(bi), dev(rm), dev(rv)
    check(gpu.ach_bn_infer(d_x.ptr, d_out.ptr, B, Cc, H * W, d_sc.ptr, d_bi.ptr, d_rm.ptr,
                           d_rv.ptr, act, None))
    assert rel_err(d_out.numpy(), ref) < 1e-6
    assert np.array_equal(d_x.numpy(), out)
    check(gpu.ach_bn_infer(d_x.ptr, d_x.ptr, B, Cc, H * W, d_sc.ptr, d_bi.ptr, d_rm.ptr,
                           d_rv.ptr, act, None))
    assert np.array_equal(d_x.numpy(), d_out.numpy())
    assert np.array_equal(d_rm.numpy(), rm) and np.array_equal(d_rv.numpy(), rv)


@pytest.mark.parametrize("F,fsize", [(6, 27), (128, 1152), (512, 4608), (1000, 4096)])
def test_conv_bn_fold(gpu, oracle, F, fsize):
    """ach_conv_bn_fold vs the oracle's fuseConvBatchnorm: identical floats
    (both round one double result per value; at most 1 ulp apart where the
    oracle's -ffast-math build rewrites the double division)."""
    rng = np.random.default_rng(F + fsize)
    w = rng.normal(0, .1, (F, fsize)).astype(np.float32)
    b = rng.normal(0, .2, F).astype(np.float32)
    g = rng.uniform(.5, 2, F).astype(np.float32)
    m = rng.uniform(-1, 1, F).astype(np.float32)
    v = np.exp(rng.uniform(np.log(1e-6), np.log(10.), F)).astype(np.float32)
    wr, br = oracle.conv_bn_fold(w, b, g, m, v)
    d_w, d_b, d_g, d_m, d_v = dev(w), dev(b), dev(g), dev(m), dev(v)
    check(gpu.ach_conv_bn_fold(F, fsize, d_w.ptr, d_b.ptr, d_g.ptr, d_m.ptr, d_v.ptr, None))
    gw, gb = d_w.numpy(), d_b.numpy()
    ulp_w = np.abs(gw.view(np.int32).astype(np.int64) - wr.view(np.int32).astype(np.int64))
    ulp_b = np.abs(gb.view(np.int32).astype(np.int64) - br.view(np.int32).astype(np.int64))
    assert ulp_w.max() <= 1 and ulp_b.max() <= 1
    assert np.mean(ulp_w == 0) > 0.999
    assert np.array_equal(d_g.numpy(), g) and np.array_equal(d_v.numpy(), v)


def test_conv_bn_fold_errors(gpu):
    d = dev(np.zeros(8, np.float32))
    assert gpu.ach_conv_bn_fold(0, 4, d.ptr, d.ptr, d.ptr, d.ptr, d.ptr, None) == aetcnn.ACH_EINVAL
    assert gpu.ach_conv_bn_fold(2, 4, None, d.ptr, d.ptr, d.ptr, d.ptr, None) == aetcnn.ACH_EINVAL


@pytest.mark.parametrize("B,Cc,H,W", [(8, 16, 32, 32), (4, 24, 13, 13), (128, 32, 8, 8)])
@pytest.mark.parametrize("act", [aetcnn.LINEAR, aetcnn.LEAKY, aetcnn.RELU])
def test_bn_bwd(gpu, oracle, B, Cc, H, W, act):
    out, sc, bi, rm, rv = _bn_inputs(B, Cc, H, W, 7 * B + Cc + act)
    f = oracle.bn_forward(out, sc, bi, rm, rv)
    y = oracle.activate(f["out"], act)
    rng = np.random.default_rng(B * Cc + act)
    delta = rng.standard_normal(out.shape).astype(np.float32)
    su0 = rng.standard_normal(Cc).astype(np.float32) * 0.1
    d_after_act = oracle.gradient(y, act, delta)
    ref = oracle.bn_backward(d_after_act, f["x"], f["xn"], f["mean"], f["var"], sc, su0)
    d_delta, d_x = dev(delta), dev(f["x"])
    d_m, d_v, d_sc, d_bi, d_su = dev(f["mean"]), dev(f["var"]), dev(sc), dev(bi), dev(su0)
    d_md, d_vd = D(Cc), D(Cc)
    ws = gpu.ach_bn_workspace(B, Cc, H * W)
    d_ws = D(ws // 4 + 1)
    check(gpu.ach_bn_bwd(d_delta.ptr, B, Cc, H * W, d_x.ptr, None, d_m.ptr, d_v.ptr, d_sc.ptr,
                         d_bi.ptr, d_su.ptr, d_md.ptr, d_vd.ptr, act, d_ws.ptr, ws, None))
    assert rel_err(d_su.numpy(), ref["scale_updates"]) < TOL
    assert rel_err(d_md.numpy(), ref["mean_delta"]) < TOL
    assert rel_err(d_vd.numpy(), ref["var_delta"]) < TOL
    assert rel_err(d_delta.numpy(), ref["delta"]) < TOL


# ---------------------------------------------------------------------------
@pytest.mark.parametrize("act", [aetcnn.LEAKY, aetcnn.RELU, aetcnn.LINEAR, aetcnn.LOGISTIC])
def test_activation_bit_exact(gpu, oracle, act):
    rng = np.random.default_rng(act)
    x = rng.standard_normal(100003).astype(np.float32) * 3
    x[:5] = [0.0, -0.0, 1e-38, -1e-38, 2.5]
    ref = oracle.activate(x, act)
    d = dev(x)
    check(gpu.ach_activate(d.ptr, x.size, act, None))
    got = d.numpy()
    if act == aetcnn.LOGISTIC:
        assert rel_err(got, ref) < 1e-6
    else:
        assert np.array_equal(got, ref)
    delta = rng.standard_normal(x.size).astype(np.float32)
    gref = oracle.gradient(ref, act, delta)
    dd = dev(delta)
    check(gpu.ach_gradient(dev(ref).ptr, x.size, act, dd.ptr, None))
    if act == aetcnn.LOGISTIC:  # (1-y)*y*d: FMA contraction may differ by 1 ulp
        assert rel_err(dd.numpy(), gref) < 1e-6
    else:
        assert np.array_equal(dd.numpy(), gref)


@pytest.mark.parametrize("B,Cc,H,W,size,stride,pad", [
    (4, 3, 32, 32, 2, 2, 1),      # darknet default padding = size-1
    (2, 5, 55, 55, 3, 2, 0),      # AlexNet overlapping 3x3/2
    (2, 4, 13, 13, 3, 2, 2),
    (3, 7, 13, 13, 3, 2, 0),      # 6 planes per workgroup, partial last workgroup
    (2, 5, 27, 27, 3, 2, 0),      # one 729-pixel plane per workgroup
    (2, 3, 50, 50, 3, 2, 2),      # LDS-staged forward with padded windows (625 outputs)
    (3, 5, 33, 65, 3, 2, 0),      # staged forward, 2 planes per workgroup, partial last
    (3, 2, 7, 9, 2, 1, 1),
    (2, 3, 16, 16, 2, 2, 0),
    (2, 3, 8, 12, 2, 2, 1),       # 2x2/2 fast path, non-square
    (1, 2, 6, 6, 2, 2, 1),        # W % 4 != 0: generic kernel
    (1, 2, 140, 140, 3, 2, 0),    # output plane above the LDS-staged limit
    (2, 3, 150, 40, 2, 1, 1),     # generic window, plane above the limit
])
def test_maxpool_bit_exact(gpu, oracle, B, Cc, H, W, size, stride, pad):
    rng = np.random.default_rng(H * W + size)
    # small integers produce many ties: first max in scan order must win
    x = rng.integers(-3, 4, (B, Cc, H, W)).astype(np.float32)
    out, idx = oracle.maxpool_forward(x, size, stride, pad)
    dx, dout, didx = dev(x), D(out.shape), D(out.shape, np.int32)
    check(gpu.ach_maxpool_fwd(dx.ptr, B, Cc, H, W, size, stride, pad, dout.ptr, didx.ptr, None))
    assert np.array_equal(dout.numpy(), out)
    assert np.array_equal(didx.numpy(), idx)
    g = rng.standard_normal(out.shape).astype(np.float32)
    g.reshape(-1)[::7] = -0.0  # +0 + -0 must give +0, as on the zeroed reference delta
    din0 = rng.standard_normal(x.shape).astype(np.float32)
    ref = oracle.maxpool_backward(g, idx, din0)
    ddin = dev(din0)
    dg = dev(g)
    check(gpu.ach_maxpool_bwd(dg.ptr, didx.ptr, B, Cc, H, W, size, stride, pad, ddin.ptr, 1,
                              None))
    assert np.array_equal(ddin.numpy(), ref)
    # accumulate = 0: delta_in is written, never read (NaN contents ignored)
    ref0 = oracle.maxpool_backward(g, idx, np.zeros_like(x))
    ddin0 = dev(np.full(x.shape, np.nan, np.float32))
    check(gpu.ach_maxpool_bwd(dg.ptr, didx.ptr, B, Cc, H, W, size, stride, pad, ddin0.ptr, 0,
                              None))
    got0 = ddin0.numpy()
    assert np.array_equal(got0.view(np.uint32), ref0.view(np.uint32))


@pytest.mark.parametrize("B,Cc,H,W,size,stride,pad", [
    (2, 5, 55, 55, 3, 2, 0),      # LDS-staged plane kernel
    (3, 7, 13, 13, 3, 2, 0),      # several planes per workgroup
    (4, 3, 32, 32, 2, 2, 1),      # 2x2/2 fast path (float4 y loads)
    (1, 2, 140, 140, 3, 2, 0),    # gather kernel (plane above the LDS limit)
    (3, 2, 7, 9, 2, 1, 1),        # generic window
])
@pytest.mark.parametrize("act", [aetcnn.RELU, aetcnn.LEAKY, aetcnn.LOGISTIC])
def test_maxpool_bwd_act_fused(gpu, oracle, B, Cc, H, W, size, stride, pad, act):
    """ach_maxpool_bwd_act == ach_maxpool_bwd then ach_gradient, bit for bit."""
    rng = np.random.default_rng(H + 7 * act)
    x = rng.integers(-3, 4, (B, Cc, H, W)).astype(np.float32)
    out, idx = oracle.maxpool_forward(x, size, stride, pad)
    y = rng.standard_normal(x.shape).astype(np.float32)
    if act == aetcnn.LOGISTIC:
        y = 1 / (1 + np.exp(-y)).astype(np.float32)
    y.reshape(-1)[::5] = 0.0
    g = rng.standard_normal(out.shape).astype(np.float32)
    dg, di, dy_ = dev(g), dev(idx.astype(np.int32)), dev(y)
    ref = dev(np.zeros(x.shape, np.float32))
    check(gpu.ach_maxpool_bwd(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad, ref.ptr, 0, None))
    check(gpu.ach_gradient(dy_.ptr, x.size, act, ref.ptr, None))
    got = dev(np.full(x.shape, np.nan, np.float32))
    check(gpu.ach_maxpool_bwd_act(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad, got.ptr, 0,
                                  dy_.ptr, act, None))
    a, b = ref.numpy(), got.numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert gpu.ach_maxpool_bwd_act(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad, got.ptr, 0,
                                   None, act, None) == aetcnn.ACH_EINVAL


@pytest.mark.parametrize("B,Cc,H,W,size,stride,pad", [
    (3, 5, 55, 55, 3, 2, 0),      # AlexNet pool 1: one plane per workgroup
    (3, 7, 27, 27, 3, 2, 0),      # pool 2
    (5, 7, 13, 13, 3, 2, 0),      # pool 5: six planes per workgroup, partial last
    (2, 3, 20, 20, 2, 2, 1),      # 2x2/2 through the staged kernel
])
@pytest.mark.parametrize("act", [aetcnn.RELU, aetcnn.LEAKY, aetcnn.LINEAR])
def test_maxpool_bwd_act_planes(gpu, oracle, B, Cc, H, W, size, stride, pad, act):
    """ach_maxpool_bwd_act_planes writes the delta of ach_maxpool_bwd_act
    bit for bit and each (image, channel) plane's sum of it in double; the
    bias gradient from those sums (ach_bias_grad_planes) equals
    ach_bias_grad over the delta (BiasData.c:40-57)."""
    rng = np.random.default_rng(H + 3 * act)
    x = rng.integers(-3, 4, (B, Cc, H, W)).astype(np.float32)
    out, idx = oracle.maxpool_forward(x, size, stride, pad)
    y = rng.standard_normal(x.shape).astype(np.float32)
    g = rng.standard_normal(out.shape).astype(np.float32)
    dg, di, dy_ = dev(g), dev(idx.astype(np.int32)), dev(y)
    ref = dev(np.zeros(x.shape, np.float32))
    check(gpu.ach_maxpool_bwd_act(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad, ref.ptr, 0,
                                  dy_.ptr, act, None))
    got = dev(np.full(x.shape, np.nan, np.float32))
    ps = dev(np.full(B * Cc, np.nan))
    check(gpu.ach_maxpool_bwd_act_planes(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad, got.ptr,
                                         dy_.ptr, act, ps.ptr, None))
    a, b = ref.numpy(), got.numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    sums = b.astype(np.float64).sum(axis=(2, 3)).reshape(-1)
    assert np.allclose(ps.numpy(), sums, rtol=1e-12, atol=1e-12)
    u0 = rng.standard_normal(Cc).astype(np.float32)
    ua, ub = dev(u0), dev(u0)
    ws = gpu.ach_bias_grad_workspace(B, Cc, H * W)
    dws = D(ws // 4 + 1)
    check(gpu.ach_bias_grad(ua.ptr, got.ptr, B, Cc, H * W, dws.ptr, ws, None))
    check(gpu.ach_bias_grad_planes(ub.ptr, ps.ptr, B, Cc, None))
    assert rel_err(ub.numpy(), ua.numpy()) < 1e-7


@pytest.mark.parametrize("B,Cc,H,W,size,stride,pad,sums", [
    (3, 5, 55, 55, 3, 2, 0, True),    # AlexNet pool 1
    (3, 7, 27, 27, 3, 2, 0, True),    # pool 2
    (5, 7, 13, 13, 3, 2, 0, True),    # pool 5: six planes per workgroup
    (2, 3, 20, 20, 2, 2, 1, True),    # padded 2x2/2 windows
    (4, 8, 8, 8, 2, 2, 1, False),     # 16 planes per workgroup: no plane sums
    (2, 3, 9, 11, 3, 1, 1, False),    # overlapping stride-1 windows, odd sizes
])
@pytest.mark.parametrize("act", [aetcnn.RELU, aetcnn.LEAKY])
def test_maxpool_bwd_act_pooled(gpu, oracle, B, Cc, H, W, size, stride, pad, sums, act):
    """ach_maxpool_bwd_act_pooled takes the activation gradient from the
    pool's output: the delta (and plane sums) of ach_maxpool_bwd_act(_planes)
    with the layer's output, bit for bit.  The layer's output is an
    activated tensor with ties (integers, zeros from relu)."""
    rng = np.random.default_rng(H + 5 * act + size)
    z = rng.integers(-4, 5, (B, Cc, H, W)).astype(np.float32)
    x = np.where(z > 0, z, np.float32(0) if act == aetcnn.RELU else np.float32(0.1) * z)
    x = x.astype(np.float32)
    out, idx = oracle.maxpool_forward(x, size, stride, pad)
    g = rng.standard_normal(out.shape).astype(np.float32)
    dg, di, dx, dout = dev(g), dev(idx.astype(np.int32)), dev(x), dev(out)
    ref = dev(np.zeros(x.shape, np.float32))
    check(gpu.ach_maxpool_bwd_act(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad, ref.ptr, 0,
                                  dx.ptr, act, None))
    got = dev(np.full(x.shape, np.nan, np.float32))
    ps = dev(np.full(B * Cc, np.nan)) if sums else None
    check(gpu.ach_maxpool_bwd_act_pooled(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad, got.ptr,
                                         dout.ptr, act, ps.ptr if sums else None, None))
    a, b = ref.numpy(), got.numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    if sums:
        ps2 = dev(np.full(B * Cc, np.nan))
        check(gpu.ach_maxpool_bwd_act_planes(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad,
                                             ref.ptr, dx.ptr, act, ps2.ptr, None))
        assert np.array_equal(ps.numpy().view(np.uint64), ps2.numpy().view(np.uint64))
    assert gpu.ach_maxpool_bwd_act_pooled(dg.ptr, di.ptr, B, Cc, H, W, size, stride, pad,
                                          got.ptr, dout.ptr, aetcnn.LOGISTIC, None,
                                          None) == aetcnn.ACH_EINVAL


def test_maxpool_bwd_act_planes_unsupported(gpu):
    """Small input planes (more than 8 per workgroup) keep the separate bias
    gradient: nothing is launched."""
    B, Cc, H, W = 4, 8, 8, 8  # 16 planes of 64 pixels per workgroup
    g, idx = dev(np.zeros(B * Cc * 16, np.float32)), dev(np.zeros(B * Cc * 16, np.int32))
    din, ps = dev(np.zeros(B * Cc * H * W, np.float32)), dev(np.zeros(B * Cc))
    assert gpu.ach_maxpool_bwd_act_planes(g.ptr, idx.ptr, B, Cc, H, W, 2, 2, 1, din.ptr, None,
                                          aetcnn.LINEAR, ps.ptr, None) == aetcnn.ACH_EUNSUPPORTED


@pytest.mark.parametrize("B,n,sp", [(3, 5, 169), (2, 4, 3025), (4, 3, 130), (2, 3, 2000)])
@pytest.mark.parametrize("act", [aetcnn.RELU, aetcnn.LEAKY, aetcnn.LOGISTIC, aetcnn.LINEAR])
def test_gradient_planes(gpu, B, n, sp, act):
    """ach_gradient_planes: the products of ach_gradient bit for bit, plus
    the per-plane sums of the result."""
    rng = np.random.default_rng(sp + act)
    y = rng.standard_normal((B, n, sp)).astype(np.float32)
    if act == aetcnn.LOGISTIC:
        y = (1 / (1 + np.exp(-y))).astype(np.float32)
    d = rng.standard_normal(y.shape).astype(np.float32)
    dy_, da, db = dev(y), dev(d), dev(d)
    check(gpu.ach_gradient(dy_.ptr, y.size, act, da.ptr, None))
    ps = dev(np.full(B * n, np.nan))
    check(gpu.ach_gradient_planes(dy_.ptr, B, n, sp, act, db.ptr, ps.ptr, None))
    a, b = da.numpy(), db.numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.allclose(ps.numpy(), b.astype(np.float64).sum(axis=2).reshape(-1), rtol=1e-12,
                       atol=1e-12)


@pytest.mark.parametrize("B,Cc,H,W,size,stride,pad", [
    (4, 3, 32, 32, 2, 2, 1),      # 2x2/2 kernels: mask applied inside
    (2, 5, 55, 55, 3, 2, 0),      # other windows: two steps inside the call
])
def test_maxpool_dropout_fused(gpu, B, Cc, H, W, size, stride, pad):
    """ach_maxpool_fwd_dropout == ach_maxpool_fwd + ach_dropout_fwd on the
    output; ach_maxpool_bwd_dropout == ach_dropout_bwd on delta_out +
    ach_maxpool_bwd; bit for bit."""
    rng = np.random.default_rng(H + size)
    x = rng.standard_normal((B, Cc, H, W)).astype(np.float32)
    OH = gpu.ach_maxpool_out(H, size, stride, pad)
    OW = gpu.ach_maxpool_out(W, size, stride, pad)
    n = B * Cc * OH * OW
    p, seed, it, layer = 0.5, 77, 5, 4
    dx = dev(x)
    o0, i0 = D((n,)), D((n,), np.int32)
    check(gpu.ach_maxpool_fwd(dx.ptr, B, Cc, H, W, size, stride, pad, o0.ptr, i0.ptr, None))
    check(gpu.ach_dropout_fwd(o0.ptr, n, p, seed, it, layer, None))
    o1, i1 = D((n,)), D((n,), np.int32)
    check(gpu.ach_maxpool_fwd_dropout(dx.ptr, B, Cc, H, W, size, stride, pad, o1.ptr, i1.ptr, p,
                                      seed, it, layer, None))
    assert np.array_equal(o0.numpy().view(np.uint32), o1.numpy().view(np.uint32))
    assert np.array_equal(i0.numpy(), i1.numpy())
    g = rng.standard_normal(n).astype(np.float32)
    gd = dev(g)
    check(gpu.ach_dropout_bwd(gd.ptr, n, p, seed, it, layer, None))
    ref = D(x.shape)
    check(gpu.ach_maxpool_bwd(gd.ptr, i0.ptr, B, Cc, H, W, size, stride, pad, ref.ptr, 0, None))
    got = dev(np.full(x.shape, np.nan, np.float32))
    check(gpu.ach_maxpool_bwd_dropout(dev(g).ptr, i0.ptr, B, Cc, H, W, size, stride, pad,
                                      got.ptr, 0, p, seed, it, layer, None))
    assert np.array_equal(ref.numpy().view(np.uint32), got.numpy().view(np.uint32))
    assert gpu.ach_maxpool_fwd_dropout(dx.ptr, B, Cc, H, W, size, stride, pad, o0.ptr, i0.ptr,
                                       1.0, seed, it, layer, None) == aetcnn.ACH_EINVAL


def test_avgpool_bit_exact(gpu, oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((128, 10, 8, 8)).astype(np.float32)
    ref = oracle.avgpool_forward(x)
    dout = D(ref.shape)
    check(gpu.ach_avgpool_fwd(dev(x).ptr, 128, 10, 64, dout.ptr, None))
    assert np.array_equal(dout.numpy(), ref)
    g = rng.standard_normal(ref.shape).astype(np.float32)
    din0 = rng.standard_normal(x.shape).astype(np.float32)
    refb = oracle.avgpool_backward(g, x.shape, din0)
    ddin = dev(din0)
    check(gpu.ach_avgpool_bwd(dev(g).ptr, 128, 10, 64, ddin.ptr, None))
    assert np.array_equal(ddin.numpy(), refb)


@pytest.mark.parametrize("B,n,groups", [(128, 10, 1), (512, 1000, 1), (7, 12, 3),
                                        (5, 300, 1), (3, 1536, 3)])  # workgroup per row
def test_softmax_xent(gpu, oracle, B, n, groups):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((B, n)) * 3).astype(np.float32)
    labels = rng.integers(0, n // groups, (B, groups))
    truth = np.zeros((B, n), np.float32)
    for b in range(B):
        for g in range(groups):
            truth[b, g * (n // groups) + labels[b, g]] = 1
    out, delta, err, cost = oracle.softmax_xent(x, truth, groups)
    dout, ddelta, derr, dcost = D(x.shape), D(x.shape), D(x.shape), D(1)
    ws = gpu.ach_softmax_workspace(B, groups)
    dws = D(ws // 4 + 1)
    check(gpu.ach_softmax_xent(dev(x).ptr, B, n, groups, 1.0, dev(truth).ptr, dout.ptr,
                               ddelta.ptr, derr.ptr, dcost.ptr, dws.ptr, ws, None))
    got = dout.numpy()
    assert rel_err(got, out) < 1e-6
    assert rel_err(ddelta.numpy(), delta) < 1e-6
    assert rel_err(derr.numpy(), err) < 1e-6
    assert abs(dcost.numpy()[0] - cost) <= 1e-5 * abs(cost)
    # label predictions bit-exact
    assert np.array_equal(got.reshape(B * groups, -1).argmax(1),
                          out.reshape(B * groups, -1).argmax(1))


def test_dropout_mask_bit_exact(gpu, oracle):
    n = 1 << 20
    for (p, seed, it, layer) in [(0.5, 1, 0, 7), (0.2, 12345, 99, 3), (0.0, 5, 1, 1)]:
        ref = oracle.dropout_mask_scale(n, p, seed, it, layer)
        d = dev(np.ones(n, np.float32))
        check(gpu.ach_dropout_fwd(d.ptr, n, p, seed, it, layer, None))
        assert np.array_equal(d.numpy(), ref)
        check(gpu.ach_dropout_bwd(d.ptr, n, p, seed, it, layer, None))
        assert np.array_equal(d.numpy(), oracle.dropout_mask_scale(n, p, seed, it, layer) * ref)
    assert gpu.ach_dropout_uniform(3, 4, 5, 6) == oracle.lib().or_dropout_uniform(3, 4, 5, 6)


def test_conv_update(gpu, oracle):
    rng = np.random.default_rng(11)
    nw, n = 10007, 64
    w, dw = rng.standard_normal(nw).astype(np.float32), rng.standard_normal(nw).astype(np.float32)
    b, db = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    s, ds = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    ref = oracle.conv_update(w, dw, b, db, s, ds, 128, 0.1, 0.9, 5e-4)
    arrs = [dev(a) for a in (w, dw, b, db, s, ds)]
    check(gpu.ach_conv_update(nw, arrs[0].ptr, arrs[1].ptr, n, arrs[2].ptr, arrs[3].ptr,
                              arrs[4].ptr, arrs[5].ptr, 128, 0.1, 0.9, 5e-4, None))
    for a, r in zip(arrs, ref):
        assert rel_err(a.numpy(), r) < 1e-6


@pytest.mark.parametrize("n", [1, 64, 1000, 4099])
def test_conv_update_pair_matches_sgd(gpu, n):
    """ach_conv_update with BN scales (biases and scales in one launch)
    equals ach_sgd_update on each array, bit for bit."""
    rng = np.random.default_rng(n)
    b, db = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    s, ds = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    got = [dev(a) for a in (b, db, s, ds)]
    ref = [dev(a) for a in (b, db, s, ds)]
    check(gpu.ach_conv_update(0, None, None, n, got[0].ptr, got[1].ptr, got[2].ptr, got[3].ptr,
                              64, 0.1, 0.9, 5e-4, None))
    lc = np.float32(0.1) / np.float32(64)
    check(gpu.ach_sgd_update(n, ref[0].ptr, ref[1].ptr, 0.0, lc, 0.9, None))
    check(gpu.ach_sgd_update(n, ref[2].ptr, ref[3].ptr, 0.0, lc, 0.9, None))
    for a, r in zip(got, ref):
        assert np.array_equal(a.numpy().view(np.uint32), r.numpy().view(np.uint32))


@pytest.mark.parametrize("B,n,sp", [(16, 10, 64), (8, 300, 1), (5, 40, 12), (9, 6, 169)])
def test_bias_ops(gpu, oracle, B, n, sp):
    """add_bias bit-exact; bias gradient (large planes: two-pass partials;
    planes of <= 16 positions, e.g. FC outputs: one thread per channel)
    within 1e-5 of the oracle's sums."""
    rng = np.random.default_rng(12 + B + n + sp)
    out = rng.standard_normal((B, n, sp)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    ref = out.copy()
    oracle.lib().or_add_bias(oracle.P(ref), oracle.P(bias), B, n, sp)
    d = dev(out)
    check(gpu.ach_add_bias(d.ptr, dev(bias).ptr, B, n, sp, None))
    assert np.array_equal(d.numpy(), ref)
    upd = rng.standard_normal(n).astype(np.float32)
    refu = upd.copy()
    oracle.lib().or_bias_grad(oracle.P(refu), oracle.P(out), B, n, sp)
    du = dev(upd)
    ws = gpu.ach_bias_grad_workspace(B, n, sp)
    dws = dev(np.zeros(ws // 4 + 1, np.float32))
    check(gpu.ach_bias_grad(du.ptr, dev(out).ptr, B, n, sp, dws.ptr, ws, None))
    assert rel_err(du.numpy(), refu) < 1e-5


@pytest.mark.parametrize("shape", [
    (2, 128, 16, 16, 256, 3, 1, 1),   # no split (GEMM epilogue)
    (2, 256, 8, 8, 512, 3, 1, 1),     # split K (reduction epilogue)
    (2, 128, 32, 32, 128, 3, 1, 1),   # no split (GEMM epilogue)
    (2, 3, 32, 32, 128, 3, 1, 1),     # shallow im2col kernel
    (2, 1, 12, 10, 70, 5, 1, 2),      # shallow im2col kernel, 5x5, ragged M
    (3, 5, 9, 7, 10, 3, 1, 1),        # scalar loaders, ragged tiles
    (2, 96, 9, 9, 80, 5, 1, 2),       # padded-tap 5x5, 96-row tiles
    (2, 16, 13, 13, 24, 5, 1, 2),
    (2, 3, 35, 35, 8, 11, 4, 0),      # row-tap loaders (11x11, no padding), stride 4
    (2, 3, 35, 35, 96, 11, 4, 0),     # row-tap loaders, 96-row tiles
    (4, 3, 227, 227, 96, 11, 4, 0),   # AlexNet conv1 at batch 4
    (2, 3, 35, 35, 96, 7, 4, 0),      # generic loader, 96-row tiles
    (2, 512, 8, 8, 10, 1, 1, 0),      # 1x1
    (128, 256, 8, 8, 512, 3, 1, 1),   # K split in two inside one workgroup
    (8, 64, 1, 1, 48, 1, 1, 0),       # fully connected GEMM
    (4, 300, 1, 1, 64, 1, 1, 0),      # fully connected, split K
    (16, 2048, 1, 1, 8192, 1, 1, 0),  # fully connected, pairs of K slices per workgroup
], ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("act", [aetcnn.LEAKY, aetcnn.RELU, aetcnn.LINEAR, aetcnn.LOGISTIC])
def test_conv_fwd_bias_act_fused(gpu, shape, act):
    """ach_conv_fwd_bias_act_prepared equals ach_conv_fwd_prepared +
    ach_add_bias + ach_activate bit for bit (with and without a bias)."""
    B, Cc, H, W, F, k, s, p = shape
    x, w, dy = _conv_inputs(shape, 11)
    rng = np.random.default_rng(12)
    bias = rng.standard_normal(F).astype(np.float32)
    d = conv_desc(*shape)
    ws = gpu.ach_conv_fwd_workspace(C.byref(d))
    dws = dev(np.zeros(ws // 4 + 64, np.float32))
    dx_, dw_, db = dev(x), dev(w), dev(bias)
    wt = dev(np.zeros(w.size, np.float32))
    job = aetcnn.FilterJob(d, dw_.ptr, wt.ptr, None)
    check(gpu.ach_conv_prepare_filters(1, C.byref(job), None))
    if gpu.ach_conv_is_fully_connected(C.byref(d)):
        wt = dw_  # the forward reads W itself
    oh, ow = gpu.ach_conv_out_h(C.byref(d)), gpu.ach_conv_out_w(C.byref(d))
    for bptr in (db.ptr, None):
        y0, y1 = D(dy.shape), D(dy.shape)
        check(gpu.ach_conv_fwd_prepared(C.byref(d), dx_.ptr, wt.ptr, y0.ptr, dws.ptr, ws, None))
        if bptr is not None:
            check(gpu.ach_add_bias(y0.ptr, bptr, B, F, oh * ow, None))
        check(gpu.ach_activate(y0.ptr, int(np.prod(dy.shape)), act, None))
        check(gpu.ach_conv_fwd_bias_act_prepared(C.byref(d), dx_.ptr, wt.ptr, bptr, act, y1.ptr,
                                                 dws.ptr, ws, None))
        a, b = y0.numpy(), y1.numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (shape, act, bptr is None)
    assert gpu.ach_conv_fwd_bias_act_prepared(C.byref(d), dx_.ptr, wt.ptr, db.ptr, 2, y1.ptr,
                                              dws.ptr, ws, None) == aetcnn.ACH_EUNSUPPORTED


@pytest.mark.parametrize("shape", [
    (512, 3, 16, 8, 128, 3, 1, 1),    # 128 filters per workgroup, 4 tiles per wave
    (256, 3, 32, 32, 48, 3, 1, 1),    # 64 filters per workgroup, 8 tiles per wave, ragged M
    (512, 3, 32, 32, 16, 3, 1, 1),    # 32 filters per workgroup, 8 tiles per wave
    (256, 3, 34, 34, 64, 3, 1, 0),    # 32-wide output rows without padding (row tiles)
    (512, 1, 16, 16, 40, 5, 1, 2),    # 5x5 (kernel size at run time), 4 tiles per wave
], ids=lambda s: "x".join(map(str, s)))
def test_conv_fwd_shallow_tile_counts(gpu, oracle, shape):
    """The patch-staged shallow-im2col forward walks 4 or 8 tiles per wave
    only when the grid is large: forward against the oracle, and the fused
    bias + leaky epilogue bit-equal to the separate passes."""
    B, Cc, H, W, F, k, s, p = shape
    x, w, _ = _conv_inputs(shape, 21)
    ref = oracle.conv_forward(x, w, F, k, s, p)
    d = conv_desc(*shape)
    ws = gpu.ach_conv_fwd_workspace(C.byref(d))
    dws = dev(np.zeros(ws // 4 + 64, np.float32))
    dx, dw = dev(x), dev(w)
    y = D(ref.shape)
    check(gpu.ach_fill(y.ptr, ref.size, 123.0, None))  # must be overwritten
    check(gpu.ach_conv_fwd(C.byref(d), dx.ptr, dw.ptr, y.ptr, dws.ptr, ws, None))
    assert rel_err(y.numpy(), ref) < TOL
    bias = dev(np.random.default_rng(22).standard_normal(F).astype(np.float32))
    wt = dev(np.zeros(w.size, np.float32))
    job = aetcnn.FilterJob(d, dw.ptr, wt.ptr, None)
    check(gpu.ach_conv_prepare_filters(1, C.byref(job), None))
    y0, y1 = D(ref.shape), D(ref.shape)
    oh, ow = gpu.ach_conv_out_h(C.byref(d)), gpu.ach_conv_out_w(C.byref(d))
    check(gpu.ach_conv_fwd_prepared(C.byref(d), dx.ptr, wt.ptr, y0.ptr, dws.ptr, ws, None))
    check(gpu.ach_add_bias(y0.ptr, bias.ptr, B, F, oh * ow, None))
    check(gpu.ach_activate(y0.ptr, ref.size, aetcnn.LEAKY, None))
    check(gpu.ach_conv_fwd_bias_act_prepared(C.byref(d), dx.ptr, wt.ptr, bias.ptr, aetcnn.LEAKY,
                                             y1.ptr, dws.ptr, ws, None))
    assert np.array_equal(y0.numpy().view(np.uint32), y1.numpy().view(np.uint32))


@pytest.mark.parametrize("shape", [
    (2, 128, 16, 16, 256, 3, 1, 1),   # 3x3, 256-row tiles, split K
    (3, 5, 9, 7, 10, 3, 1, 1),
    (2, 16, 13, 13, 24, 5, 1, 2),     # generic kernel size
    (2, 512, 8, 8, 10, 1, 1, 0),      # 1x1: the flipped filter is W itself
    (3, 8, 6, 6, 40, 6, 1, 0),        # kernel covers the input: a 1x1 of the flattened input
], ids=lambda s: "x".join(map(str, s)))
def test_conv_prepared_filters(gpu, shape):
    """ach_conv_prepare_filters + the _prepared entry points give the same
    bits as ach_conv_fwd / ach_conv_bwd_data (same kernels, same layouts)."""
    B, Cc, H, W, F, k, s, p = shape
    x, w, dy = _conv_inputs(shape, 3)
    d = conv_desc(*shape)
    ws = max(gpu.ach_conv_fwd_workspace(C.byref(d)), gpu.ach_conv_bwd_data_workspace(C.byref(d)))
    dws = dev(np.zeros(ws // 4 + 64, np.float32))
    dx_, dw_, ddy = dev(x), dev(w), dev(dy)
    wt, wft = dev(np.zeros(w.size, np.float32)), dev(np.full(w.size, np.nan, np.float32))
    job = aetcnn.FilterJob(d, dw_.ptr, wt.ptr, wft.ptr)
    check(gpu.ach_conv_prepare_filters(1, C.byref(job), None))
    fc = gpu.ach_conv_is_fully_connected(C.byref(d))
    if fc:  # no k-major copy: the forward reads W itself
        assert not wt.numpy().any()
    y0, y1 = D(dy.shape), D(dy.shape)
    check(gpu.ach_conv_fwd(C.byref(d), dx_.ptr, dw_.ptr, y0.ptr, dws.ptr, ws, None))
    check(gpu.ach_conv_fwd_prepared(C.byref(d), dx_.ptr, dw_.ptr if fc else wt.ptr, y1.ptr,
                                    dws.ptr, ws, None))
    assert np.array_equal(y0.numpy(), y1.numpy())
    g0, g1 = D(x.shape), D(x.shape)
    check(gpu.ach_conv_bwd_data(C.byref(d), ddy.ptr, dw_.ptr, g0.ptr, dws.ptr, ws, None))
    check(gpu.ach_conv_bwd_data_prepared(C.byref(d), ddy.ptr, dw_.ptr, wft.ptr, g1.ptr,
                                         dws.ptr, ws, None))
    assert np.array_equal(g0.numpy(), g1.numpy())
