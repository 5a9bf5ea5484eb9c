"""Pins the CPU oracle (oracle/liboracle.so) against what the mathematics
fixes, independently of how the oracle is written: double-precision brute
force, adjoint identities, closed forms, textbook gradients, finite
differences and published known-answer values.  The reference ships no
golden vectors (it has no tests), so these checks are the pin.  CPU only."""
import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_err

LEAKY, RELU, LINEAR = 7, 1, 3


from refs64 import conv_ref, dgrad_ref, wgrad_ref  # noqa: E402


# ---- GEMM --------------------------------------------------------------------
@pytest.mark.parametrize("TA,TB", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_vs_float64(TA, TB):
    rng = np.random.default_rng(TA * 2 + TB)
    M, N, K = 13, 17, 19
    A = rng.standard_normal((K, M) if TA else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if TB else (K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    got = O.gemm(TA, TB, M, N, K, 0.75, A, A.shape[1], B, B.shape[1], 0.5, C0, N)
    a = A.T if TA else A
    b = B.T if TB else B
    ref = 0.75 * a.astype(np.float64) @ b.astype(np.float64) + 0.5 * C0
    assert rel_err(got, ref) < 1e-6


def test_gemm_parallel_is_bit_identical():
    rng = np.random.default_rng(3)
    M, N, K = 64, 100, 300
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    C0 = np.zeros((M, N), np.float32)
    O.lib().or_set_gemm_parallel(0)
    a = O.gemm(0, 0, M, N, K, 1, A, K, B, N, 1, C0, N)
    O.lib().or_set_gemm_parallel(1)
    b = O.gemm(0, 0, M, N, K, 1, A, K, B, N, 1, C0, N)
    O.lib().or_set_gemm_parallel(0)
    assert np.array_equal(a, b)


# ---- im2col / col2im -----------------------------------------------------------
@pytest.mark.parametrize("Cc,H,W,k,p,s,dl", [(2, 5, 6, 3, 1, 1, 1), (3, 9, 9, 5, 2, 2, 1),
                                             (1, 11, 11, 11, 0, 4, 1), (3, 11, 9, 3, 2, 1, 2),
                                             (2, 13, 13, 3, 3, 2, 3)])
def test_im2col_index_map_and_col2im_adjoint(Cc, H, W, k, p, s, dl):
    """Exact index map (taps at k*dilation, Im2Col.c:65-103) and col2im as
    its adjoint (Im2Col.c:155-192)."""
    rng = np.random.default_rng(k)
    im = rng.standard_normal((Cc, H, W)).astype(np.float32)
    ek = dl * (k - 1) + 1
    OH, OW = (H + 2 * p - ek) // s + 1, (W + 2 * p - ek) // s + 1
    col = np.zeros(Cc * k * k * OH * OW, np.float32)
    O.lib().or_im2col(O.P(im), Cc, H, W, k, k, p, p, s, s, dl, dl, O.P(col))
    col = col.reshape(Cc, k, k, OH, OW)
    for c in range(Cc):
        for ki in range(k):
            for kj in range(k):
                for oh in range(OH):
                    for ow in range(OW):
                        ih, iw = oh * s - p + ki * dl, ow * s - p + kj * dl
                        v = im[c, ih, iw] if 0 <= ih < H and 0 <= iw < W else 0.0
                        assert col[c, ki, kj, oh, ow] == v
    # col2im is the adjoint of im2col: <im2col(x), y> == <x, col2im(y)>
    y = rng.standard_normal(col.size).astype(np.float32)
    back = np.full((Cc, H, W), 9.0, np.float32)  # must be zeroed first
    O.lib().or_col2im(O.P(y), Cc, H, W, k, k, p, p, s, s, dl, dl, O.P(back))
    lhs = float(np.dot(col.ravel().astype(np.float64), y.astype(np.float64)))
    rhs = float(np.dot(im.ravel().astype(np.float64), back.ravel().astype(np.float64)))
    assert abs(lhs - rhs) <= 1e-5 * max(1.0, abs(lhs))


# ---- convolution ---------------------------------------------------------------
SHAPES = [(2, 3, 8, 8, 4, 3, 1, 1), (1, 4, 7, 9, 5, 5, 2, 2), (2, 2, 12, 12, 3, 11, 4, 0),
          (3, 6, 4, 4, 7, 1, 1, 0), (2, 5, 6, 6, 8, 6, 1, 0)]


@pytest.mark.parametrize("shape", SHAPES)
def test_conv_forward_vs_direct(shape):
    B, Cc, H, W, F, k, s, p = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.uniform(-1, 1, (B, Cc, H, W)).astype(np.float32)
    w = rng.standard_normal((F, Cc, k, k)).astype(np.float32)
    assert rel_err(O.conv_forward(x, w, F, k, s, p), conv_ref(x, w, s, p)) < 1e-6


@pytest.mark.parametrize("shape", SHAPES)
def test_conv_backward_vs_direct_and_adjoint(shape):
    B, Cc, H, W, F, k, s, p = shape
    rng = np.random.default_rng(sum(shape) + 1)
    x = rng.uniform(-1, 1, (B, Cc, H, W)).astype(np.float32)
    w = rng.standard_normal((F, Cc, k, k)).astype(np.float32)
    OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    dy = rng.standard_normal((B, F, OH, OW)).astype(np.float32)
    dw0 = rng.standard_normal(w.shape).astype(np.float32)
    dw, dx = O.conv_backward(x, dy, w, k, s, p, dw0=dw0)
    assert rel_err(dw, dw0 + wgrad_ref(x, dy, k, s, p)) < 1e-6  # accumulates (beta = 1)
    assert rel_err(dx, dgrad_ref(dy, w, x.shape, s, p)) < 1e-6
    # adjoint identities: <conv(x,W), dy> = <x, dgrad(dy)> = <W, wgrad(x,dy)>
    y = conv_ref(x, w, s, p)
    ip = float((y * dy).sum())
    assert abs(ip - float((x.astype(np.float64) * dx).sum())) <= 1e-5 * abs(ip) + 1e-5
    assert abs(ip - float((w.astype(np.float64) * (dw - dw0)).sum())) <= 1e-4 * abs(ip) + 1e-4


# unequal width / height strides (B, C, H, W, F, k, stride_x, stride_y, pad): the
# last is a 1x1 filter with stride_x 1, which the reference's forward would
# read as unstrided (ConvolutionalLayer.c:788 tests stride_x alone)
SHAPES_XY = [(2, 3, 9, 8, 4, 3, 2, 1, 1), (1, 2, 11, 7, 3, 5, 1, 3, 2),
             (1, 3, 12, 10, 5, 4, 3, 2, 1), (2, 2, 7, 7, 3, 1, 1, 2, 0)]


@pytest.mark.parametrize("shape", SHAPES_XY)
def test_conv_unequal_strides_vs_direct_and_adjoint(shape):
    B, Cc, H, W, F, k, sx, sy, p = shape
    rng = np.random.default_rng(sum(shape) + 7)
    x = rng.uniform(-1, 1, (B, Cc, H, W)).astype(np.float32)
    w = rng.standard_normal((F, Cc, k, k)).astype(np.float32)
    y = O.conv_forward(x, w, F, k, sx, p, stride_y=sy)
    ref = conv_ref(x, w, sx, p, sy=sy)
    assert y.shape == ref.shape == (B, F, (H + 2 * p - k) // sy + 1, (W + 2 * p - k) // sx + 1)
    assert rel_err(y, ref) < 1e-6
    dy = rng.standard_normal(y.shape).astype(np.float32)
    dw, dx = O.conv_backward(x, dy, w, k, sx, p, stride_y=sy)
    assert rel_err(dw, wgrad_ref(x, dy, k, sx, p, sy=sy)) < 1e-6
    assert rel_err(dx, dgrad_ref(dy, w, x.shape, sx, p, sy=sy)) < 1e-6
    ip = float((ref * dy).sum())
    assert abs(ip - float((x.astype(np.float64) * dx).sum())) <= 1e-5 * abs(ip) + 1e-5
    assert abs(ip - float((w.astype(np.float64) * dw).sum())) <= 1e-4 * abs(ip) + 1e-4
    # the transposed problem: strides and axes swapped give the transposed result
    yt = O.conv_forward(np.ascontiguousarray(x.transpose(0, 1, 3, 2)),
                        np.ascontiguousarray(w.transpose(0, 1, 3, 2)), F, k, sy, p, stride_y=sx)
    assert rel_err(yt.transpose(0, 1, 3, 2), ref) < 1e-6


# ---- bias ------------------------------------------------------------------------
def test_bias_add_and_grad():
    rng = np.random.default_rng(4)
    out = rng.standard_normal((3, 4, 5)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    ref = out + b[None, :, None]
    got = out.copy()
    O.lib().or_add_bias(O.P(got), O.P(b), 3, 4, 5)
    assert np.array_equal(got, ref)
    upd = np.ones(4, np.float32)
    O.lib().or_bias_grad(O.P(upd), O.P(out), 3, 4, 5)
    assert rel_err(upd, 1 + out.astype(np.float64).sum(axis=(0, 2))) < 1e-6


# ---- batch-norm ------------------------------------------------------------------
def test_bn_forward_closed_form():
    rng = np.random.default_rng(5)
    B, Cc, H, W = 6, 3, 5, 4
    out = (rng.standard_normal((B, Cc, H, W)) * 2 + 0.5).astype(np.float32)
    sc = rng.uniform(0.5, 2, Cc).astype(np.float32)
    bi = rng.standard_normal(Cc).astype(np.float32)
    rm0 = rng.standard_normal(Cc).astype(np.float32)
    rv0 = rng.uniform(0.5, 2, Cc).astype(np.float32)
    r = O.bn_forward(out, sc, bi, rm0, rv0)
    x64 = out.astype(np.float64)
    mean = x64.mean(axis=(0, 2, 3))
    var = x64.var(axis=(0, 2, 3), ddof=1)  # unbiased (NormData.c:176)
    assert rel_err(r["mean"], mean) < 1e-6
    assert rel_err(r["var"], var) < 1e-5
    assert rel_err(r["rm"], 0.9 * rm0 + 0.1 * mean) < 1e-6
    assert rel_err(r["rv"], 0.9 * rv0 + 0.1 * var) < 1e-6
    xn = (x64 - mean[None, :, None, None]) / (np.sqrt(var) + 1e-6)[None, :, None, None]
    assert np.array_equal(r["x"], out)
    assert rel_err(r["xn"], xn) < 1e-5
    assert rel_err(r["out"], xn * sc[None, :, None, None] + bi[None, :, None, None]) < 1e-5
    assert r["nan"] == 0


def test_bn_backward_textbook_gradient_and_fd():
    """dgamma = sum(delta*xn) exactly; delta' matches the textbook batch-norm
    input gradient of y = (x-mu)/sqrt(var_N + 1e-5) (biased var in the
    derivative, as the reference's /N terms), and a finite-difference check
    of that forward."""
    rng = np.random.default_rng(6)
    B, Cc, H, W = 4, 3, 6, 5
    N = B * H * W
    out = (rng.standard_normal((B, Cc, H, W)) * 1.5 + 0.3).astype(np.float32)
    sc = rng.uniform(0.5, 2, Cc).astype(np.float32)
    f = O.bn_forward(out, sc, np.zeros(Cc, np.float32))
    g = rng.standard_normal(out.shape).astype(np.float32)
    r = O.bn_backward(g, f["x"], f["xn"], f["mean"], f["var"], sc)
    assert rel_err(r["scale_updates"], (g.astype(np.float64) * f["xn"]).sum(axis=(0, 2, 3))) < 1e-6
    # textbook: for y = xhat with xhat = (x-mu)/s, s = sqrt(v + eps),
    # dL/dx = (1/s)(dyh - mean(dyh) - (x-mu)/s^2 * mean(dyh*(x-mu))), dyh = gamma*g
    x = out.astype(np.float64)
    mu = f["mean"].astype(np.float64)[None, :, None, None]
    v = f["var"].astype(np.float64)[None, :, None, None]
    s = np.sqrt(v + 1e-5)
    dyh = g * sc[None, :, None, None].astype(np.float64)
    xc = x - mu
    ref = (dyh - dyh.mean(axis=(0, 2, 3), keepdims=True)
           - xc / s ** 2 * (dyh * xc).mean(axis=(0, 2, 3), keepdims=True)) / s
    assert rel_err(r["delta"], ref) < 1e-4
    # finite differences of L(x) = sum(gamma*g*(x-mu)/sqrt(var_N(x)+1e-5)),
    # var_N with denominator N (the derivative the reference's /N terms take)
    def L(xx):
        m = xx.mean(axis=(0, 2, 3), keepdims=True)
        vn = ((xx - m) ** 2).mean(axis=(0, 2, 3), keepdims=True)
        return float((dyh * (xx - m) / np.sqrt(vn + 1e-5)).sum())
    for idx in [(0, 0, 0, 0), (1, 2, 3, 4), (3, 1, 5, 2)]:
        e = np.zeros_like(x)
        e[idx] = 1e-5
        fd = (L(x + e) - L(x - e)) / 2e-5
        # unbiased vs biased variance differ by N/(N-1): allow that much
        assert abs(fd - r["delta"][idx]) <= 5e-2 * abs(fd) / N * 10 + 2e-3 * max(1, abs(fd))


# ---- activations -------------------------------------------------------------------
def test_activations_exact():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(10001) * 3).astype(np.float32)
    x[:3] = [0.0, -0.0, -1e-30]
    leaky = np.where(x > 0, x, (0.1 * x.astype(np.float64)).astype(np.float32))
    assert np.array_equal(O.activate(x, LEAKY), leaky)
    assert np.array_equal(O.activate(x, RELU), x * (x > 0))
    assert np.array_equal(O.activate(x, LINEAR), x)
    d = rng.standard_normal(x.size).astype(np.float32)
    assert np.array_equal(O.gradient(leaky, LEAKY, d), d * np.where(leaky > 0, 1, np.float32(0.1)))
    assert np.array_equal(O.gradient(x, RELU, d), d * (x > 0))


# ---- pooling -------------------------------------------------------------------------
# (stride, stride_y): stride_y None takes or_maxpool_forward, else the _xy scan
@pytest.mark.parametrize("B,Cc,H,W,size,stride,sy,pad", [
    (2, 2, 6, 6, 2, 2, None, 1), (1, 2, 9, 9, 3, 2, None, 0), (1, 1, 5, 7, 3, 2, None, 2),
    (2, 2, 7, 9, 3, 2, 1, 2), (1, 3, 10, 6, 2, 1, 3, 1), (2, 1, 8, 8, 3, 3, 2, 0)])
def test_maxpool_brute_force(B, Cc, H, W, size, stride, sy, pad):
    rng = np.random.default_rng(H + size)
    x = rng.integers(-2, 3, (B, Cc, H, W)).astype(np.float32)  # ties
    out, idx = O.maxpool_forward(x, size, stride, pad, stride_y=sy)
    sy = stride if sy is None else sy
    assert out.shape[2:] == ((H + pad - size) // sy + 1, (W + pad - size) // stride + 1)
    OH, OW = out.shape[2:]
    off = -(pad // 2)
    flat = x.ravel()
    for b in range(B):
        for c in range(Cc):
            for i in range(OH):
                for j in range(OW):
                    best, bi = -np.finfo(np.float32).max, -1
                    for n in range(size):
                        for m in range(size):
                            h, w = off + i * sy + n, off + j * stride + m
                            if 0 <= h < H and 0 <= w < W:
                                k = ((b * Cc + c) * H + h) * W + w
                                if flat[k] > best:  # strict: first max wins
                                    best, bi = flat[k], k
                    assert out[b, c, i, j] == best and idx[b, c, i, j] == bi
    g = rng.standard_normal(out.shape).astype(np.float32)
    d0 = rng.standard_normal(x.shape).astype(np.float32)
    ref = d0.ravel().copy()
    np.add.at(ref, idx.ravel(), g.ravel())  # sequential, ascending output order
    assert np.array_equal(O.maxpool_backward(g, idx, d0).ravel(), ref)


def test_avgpool_closed_form():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 4, 5, 5)).astype(np.float32)
    assert rel_err(O.avgpool_forward(x), x.astype(np.float64).mean(axis=(2, 3))) < 1e-6
    g = rng.standard_normal((3, 4)).astype(np.float32)
    d = O.avgpool_backward(g, x.shape)
    assert rel_err(d, np.broadcast_to(g[:, :, None, None] / 25.0, x.shape)) < 1e-6


# ---- softmax + cross-entropy -----------------------------------------------------------
def test_softmax_xent_closed_form():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((5, 7)) * 4).astype(np.float32)
    t = np.zeros_like(x)
    t[np.arange(5), rng.integers(0, 7, 5)] = 1
    out, delta, err, cost = O.softmax_xent(x, t)
    x64 = x.astype(np.float64)
    p = np.exp(x64 - x64.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert rel_err(out, p) < 1e-6
    assert np.allclose(out.sum(1), 1, atol=1e-6)
    assert rel_err(delta, t - p) < 1e-6
    assert rel_err(err, np.where(t > 0, -np.log(p), 0)) < 1e-6
    assert abs(cost - float(-(t * np.log(p)).sum())) < 1e-5 * abs(cost)
    d0 = rng.standard_normal(x.shape).astype(np.float32)
    d1 = d0.copy()
    O.lib().or_softmax_backward(O.P(delta), delta.size, O.P(d1))
    assert np.array_equal(d1, d0 + delta)


# ---- dropout -------------------------------------------------------------------------------
def test_dropout_uniform_known_answer():
    # u(seed, 0, 0, 0) is the SplitMix64 finaliser of the seed; SplitMix64's
    # first output for state 0 is 0xE220A8397B1DCDAF (finaliser of the golden
    # gamma 0x9E3779B97F4A7C15), so u(gamma,0,0,0) = top 24 bits / 2^24.
    u = O.lib().or_dropout_uniform(0x9E3779B97F4A7C15, 0, 0, 0)
    assert u == (0xE220A8397B1DCDAF >> 40) / float(1 << 24)


def test_dropout_statistics_and_determinism():
    n = 1 << 20
    for p in (0.5, 0.2):
        m = O.dropout_mask_scale(n, p, 99, 3, 4)
        keep = m != 0
        assert abs((1 - keep.mean()) - p) < 3e-3
        assert np.all(m[keep] == np.float32(1.0 / (1.0 - p)))
        assert np.array_equal(m, O.dropout_mask_scale(n, p, 99, 3, 4))
        assert not np.array_equal(keep, O.dropout_mask_scale(n, p, 99, 4, 4) != 0)
        assert not np.array_equal(keep, O.dropout_mask_scale(n, p, 99, 3, 5) != 0)


# ---- SGD update ------------------------------------------------------------------------------
def test_sgd_update_closed_form_three_steps():
    rng = np.random.default_rng(10)
    nw, n = 50, 6
    w, v = rng.standard_normal(nw), rng.standard_normal(nw)
    b, vb = rng.standard_normal(n), rng.standard_normal(n)
    s, vs = rng.standard_normal(n), rng.standard_normal(n)
    W, V, Bb, VB, S, VS = (a.astype(np.float32) for a in (w, v, b, vb, s, vs))
    lr, mom, decay, batch = 0.1, 0.9, 5e-4, 128
    for _ in range(3):
        W, V, Bb, VB, S, VS = O.conv_update(W, V, Bb, VB, S, VS, batch, lr, mom, decay)
        v = v - decay * batch * w
        w = w + lr / batch * v
        v = v * mom
        b = b + lr / batch * vb
        vb = vb * mom
        s = s + lr / batch * vs
        vs = vs * mom
    for got, ref in ((W, w), (V, v), (Bb, b), (VB, vb), (S, s), (VS, vs)):
        assert rel_err(got, ref) < 1e-6


def test_weight_init_glibc_rand_known_answer():
    # glibc: srand(1); rand() == 1804289383 (the reference inits weights from
    # this default stream, WeightData.c:161 via DnnUtils.c:207)
    O.lib().or_rand_seed(1)
    u = O.lib().or_rand_uniform(-1.0, 1.0)
    assert u == np.float32(np.float32(1804289383) / np.float32(2147483647) * np.float32(2) - 1)


# ---- whole network glue ---------------------------------------------------------------------
def _tiny_nobn(onet):
    onet.conv(4, 3, 1, 1, LEAKY, 0)
    onet.maxpool(2, 2, 1)
    onet.conv(5, 1, 1, 0, LINEAR, 0)
    onet.avgpool()
    onet.softmax()


def test_network_gradient_finite_difference():
    """The network's weight_updates are -dL/dW summed over the batch
    (delta = t - p convention), with L = sum of cross-entropies."""
    B, H, W, Cc = 3, 6, 6, 2
    rng = np.random.default_rng(11)
    x = rng.random((B, Cc, H, W)).astype(np.float32)
    t = np.zeros((B, 5), np.float32)
    t[np.arange(B), rng.integers(0, 5, B)] = 1
    O.lib().or_rand_seed(3)
    net = O.OracleNet(B, H, W, Cc)
    _tiny_nobn(net)
    net.finalize()
    loss = net.forward_backward(x, t)
    g0 = net.buffer(0, 3).copy()  # weight_updates of layer 0
    w0 = net.buffer(0, 2).copy()

    def total_loss(w):
        O.lib().or_rand_seed(3)
        n2 = O.OracleNet(B, H, W, Cc)
        _tiny_nobn(n2)
        n2.finalize()
        n2.set_buffer(0, 2, w)
        val = n2.forward_backward(x, t) * B
        n2.close()
        return val

    assert abs(total_loss(w0) - loss * B) < 1e-5
    for k in (0, 7, 20):
        e = np.zeros_like(w0)
        e[k] = 2e-3
        fd = (total_loss(w0 + e) - total_loss(w0 - e)) / 4e-3
        assert abs(-fd - g0[k]) <= 3e-3 * max(1.0, abs(fd)), (k, fd, g0[k])


def test_network_forward_composes_ops():
    """or_net forward == the op functions composed by hand (pins the layer
    loop, dropout sharing and the loss = cost/batch convention)."""
    B, H, W, Cc = 4, 8, 8, 3
    rng = np.random.default_rng(12)
    x = rng.random((B, Cc, H, W)).astype(np.float32)
    t = np.zeros((B, 6), np.float32)
    t[np.arange(B), rng.integers(0, 6, B)] = 1
    O.lib().or_rand_seed(5)
    net = O.OracleNet(B, H, W, Cc)
    net.conv(5, 3, 1, 1, LEAKY, 1)
    net.maxpool(2, 2, 1)
    net.dropout(0.5)
    net.conv(6, 1, 1, 0, LINEAR, 0)
    net.avgpool()
    net.softmax()
    net.dropout_seed(77)
    net.finalize()
    w0, w3 = net.buffer(0, 2).reshape(5, 3, 3, 3), net.buffer(3, 2).reshape(6, 5, 1, 1)
    loss = net.forward_backward(x, t)
    y = O.conv_forward(x, w0, 5, 3, 1, 1)
    f = O.bn_forward(y, np.ones(5, np.float32), np.zeros(5, np.float32))
    a = O.activate(f["out"], LEAKY)
    mp, idx = O.maxpool_forward(a, 2, 2, 1)
    mp = mp * O.dropout_mask_scale(mp.size, 0.5, 77, 0, 2).reshape(mp.shape)
    z = O.conv_forward(mp, w3, 6, 1, 1, 0)
    av = O.avgpool_forward(z)
    _, _, _, cost = O.softmax_xent(av, t)
    assert abs(loss - cost / B) < 1e-6
    assert np.array_equal(net.buffer(1, 14).reshape(idx.shape), idx)


def test_bn_inference_normalize_closed_form():
    """NormData.normalizeByRoll (NormData.c:291-326): rolling statistics,
    inv = 1/(sqrt(rolling_var)+1e-6)."""
    rng = np.random.default_rng(13)
    out = rng.standard_normal((3, 4, 5, 2)).astype(np.float32)
    rm = rng.standard_normal(4).astype(np.float32)
    rv = rng.uniform(0.5, 2, 4).astype(np.float32)
    sc = rng.uniform(0.5, 2, 4).astype(np.float32)
    bi = rng.standard_normal(4).astype(np.float32)
    got = out.copy()
    O.lib().or_bn_normalize_roll(O.P(got), 3, 4, 10, O.P(rm), O.P(rv), O.P(sc), O.P(bi))
    x = out.astype(np.float64)
    ref = ((x - rm[None, :, None, None]) / (np.sqrt(rv.astype(np.float64)) + 1e-6)[None, :, None, None]
           * sc[None, :, None, None] + bi[None, :, None, None])
    assert rel_err(got, ref) < 1e-6


def test_oracle_predict_composes_inference_ops():
    """or_net_predict (NNetwork.predict, NNetwork.c:411-422) after two training
    steps equals the hand composition of the oracle's inference ops: conv,
    batch-norm on the rolling statistics, leaky, max-pool, 1x1 conv + bias,
    global avg-pool, softmax without truth -- and leaves the state alone."""
    from aetcnn import configs
    L = O.lib()
    L.or_rand_seed(3)
    B, h, w, c = configs.dims("tiny", 4)
    net = O.OracleNet(B, h, w, c)
    configs.build(net, "tiny")
    net.finalize()
    for s in range(2):
        x, truth, _ = configs.synthetic_batch("tiny", 20 + s, B)
        net.train(x, truth)
    before = {(i, k): net.buffer(i, k).copy() for i in (0, 2, 4) for k in (2, 4, 8, 9)
              if net.buffer(i, k) is not None}
    x, _, _ = configs.synthetic_batch("tiny", 99, B)
    got = net.predict(x)
    a = x
    for i, layer in enumerate(configs.CONFIGS["tiny"]["layers"]):
        kind = layer[0]
        if kind == "conv":
            F, k, st, pad, act, bn = layer[1:]
            a = O.conv_forward(a, net.buffer(i, 2).reshape(F, -1, k, k), F, k, st, pad)
            if bn:
                a = O.bn_normalize_roll(a, net.buffer(i, 8), net.buffer(i, 9),
                                        net.buffer(i, 6), net.buffer(i, 4))
            else:
                a = a + net.buffer(i, 4)[None, :, None, None]
            a = O.activate(a, act)
        elif kind == "maxpool":
            a, _ = O.maxpool_forward(a, *layer[1:])
        elif kind == "avgpool":
            a = O.avgpool_forward(a)
        elif kind == "softmax":
            a, _, _, _ = O.softmax_xent(a.reshape(B, -1), None)
    assert np.array_equal(got, a.reshape(got.shape))
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-5)
    for key, v in before.items():
        assert np.array_equal(net.buffer(*key), v), key
    net.close()


def test_conv_bn_fold_equals_conv_then_inference_affine():
    """or_conv_bn_fold (ConvolutionalLayer.c:983-1003) pinned through the
    convolution: a float64 brute-force conv with the folded filters plus the
    folded bias equals the conv with the original filters followed by the
    per-filter affine g*(y - m)/sqrt(v + 1e-5) + b.  Small variances (1e-6 ..)
    make the eps placement visible (sqrt(v + 1e-5), not sqrt(v) + 1e-6), a
    zero-mean filter would hide a dropped mean term, so the means are
    non-zero; scaling filter f by another filter's factor fails too."""
    rng = np.random.default_rng(12)
    F, Cc, k = 6, 3, 3
    x = rng.uniform(-1, 1, (2, Cc, 7, 7)).astype(np.float32)
    w = rng.normal(0, .3, (F, Cc, k, k)).astype(np.float32)
    b = rng.normal(0, .2, F).astype(np.float32)
    g = rng.uniform(.5, 2, F).astype(np.float32)
    m = rng.uniform(-1, 1, F).astype(np.float32)
    v = np.array([1e-6, 3e-6, 1e-4, .01, 1., 4.], np.float32)
    wf, bf = O.conv_bn_fold(w, b, g, m, v)
    y = conv_ref(x, w, 1, 1)
    r = np.sqrt(v.astype(np.float64) + 1e-5)[None, :, None, None]
    want = (g[None, :, None, None] * (y - m[None, :, None, None]) / r
            + b[None, :, None, None])
    got = conv_ref(x, wf.reshape(w.shape), 1, 1) + bf.astype(np.float64)[None, :, None, None]
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    # each folded value is one float rounding of the double result
    pre = g.astype(np.float64) / np.sqrt(v.astype(np.float64) + 1e-5)
    wd = w.reshape(F, -1).astype(np.float64) * pre[:, None]
    assert np.max(np.abs(wf.reshape(F, -1) - wd) / np.abs(wd)) <= 2 ** -24
    # an all-identity BN (g=1, m=0, v=1-1e-5) leaves the layer unchanged
    wi, bi = O.conv_bn_fold(w, b, np.ones(F, np.float32), np.zeros(F, np.float32),
                            np.full(F, 1 - 1e-5, np.float32))
    assert np.max(np.abs(wi - w) / np.abs(w)) <= 2 ** -23 and np.array_equal(bi, b)


def test_oracle_fused_network_predicts_like_unfused():
    """or_net_fuse_conv_batchnorm (NNetwork.c:272-288) after training: the BN
    conv layers become plain convs (biases absorb the shift) and the fused
    predictions equal the unfused inference up to the reference's eps
    difference between the fold (sqrt(v + 1e-5)) and normalizeByRoll
    (sqrt(v) + 1e-6); the predicted labels agree wherever the top two
    probabilities are apart."""
    from aetcnn import configs
    L = O.lib()
    L.or_rand_seed(5)
    B, h, w, c = configs.dims("tiny", 8)
    net = O.OracleNet(B, h, w, c)
    configs.build(net, "tiny")
    net.finalize()
    for s in range(4):
        x, truth, _ = configs.synthetic_batch("tiny", 40 + s, B)
        net.train(x, truth)
    x, _, _ = configs.synthetic_batch("tiny", 77, B)
    p0 = net.predict(x)
    net.fuse_conv_batchnorm()
    p1 = net.predict(x)
    assert rel_err(p1, p0) < 1e-3
    top2 = np.sort(p0, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1e-3
    assert np.array_equal(p1.argmax(1)[clear], p0.argmax(1)[clear])
    net.close()


def test_oracle_connected_layer():
    """or_net_add_connected: on a square input it is the convolution whose
    kernel covers the input (same initial weights, identical outputs, since
    im2col of the whole input is the flattened input in (c, h, w) order); on
    a non-square input its output equals a float64 product of the flattened
    input with the [outputs][inputs] weights."""
    L = O.lib()
    rng = np.random.default_rng(8)
    B = 4
    x = rng.uniform(-1, 1, (B, 3, 5, 5)).astype(np.float32)
    outs = []
    for connected in (True, False):
        L.or_rand_seed(11)
        net = O.OracleNet(B, 5, 5, 3)
        if connected:
            net.connected(7, 3, 0)
        else:
            net.conv(7, 5, 1, 0, 3, 0)
        net.softmax()
        net.finalize()
        net.load(x, None)
        net.layer_forward(0, 0)
        outs.append((net.buffer(0, 0).copy(), net.buffer(0, 2).copy()))
        net.close()
    assert np.array_equal(outs[0][1], outs[1][1])  # weights
    assert np.array_equal(outs[0][0], outs[1][0])  # outputs
    x2 = rng.uniform(-1, 1, (B, 2, 3, 4)).astype(np.float32)
    L.or_rand_seed(12)
    net = O.OracleNet(B, 3, 4, 2)
    net.connected(5, 3, 0)
    net.softmax()
    net.finalize()
    w = net.buffer(0, 2).reshape(5, 24).astype(np.float64)
    bias = rng.standard_normal(5).astype(np.float32)
    net.set_buffer(0, 4, bias)
    net.load(x2, None)
    net.layer_forward(0, 0)
    want = x2.reshape(B, 24).astype(np.float64) @ w.T + bias
    assert np.max(np.abs(net.buffer(0, 0).reshape(B, 5) - want)) < 1e-6
    # init: sqrt(2/inputs) * U(-1, 1)
    assert np.max(np.abs(w)) <= np.sqrt(2 / 24) + 1e-7
    net.close()
