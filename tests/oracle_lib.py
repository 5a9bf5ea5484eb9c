"""ctypes bindings for oracle/liboracle.so -- the CPU restatement of the
reference's CPU path.  Test infrastructure: used only as the checker in
tests/, by __graft_entry__.smoke() and by bench.py's CPU-baseline leg."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")

_vp, _i, _f, _sz, _u64, _u32 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint64, C.c_uint32


class OrConvShape(C.Structure):
    _fields_ = [("batch", _i), ("c", _i), ("h", _i), ("w", _i), ("n", _i), ("size", _i),
                ("stride", _i), ("pad", _i), ("stride_y", _i)]


_SIGS = {
    "or_set_gemm_parallel": (None, [_i]),
    "or_get_gemm_parallel": (_i, []),
    "or_max_threads": (_i, []),
    "or_gemm": (None, [_i, _i, _i, _i, _i, _f, _vp, _i, _vp, _i, _f, _vp, _i]),
    "or_im2col": (None, [_vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "or_col2im": (None, [_vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "or_conv_out_h": (_i, [C.POINTER(OrConvShape)]),
    "or_conv_out_w": (_i, [C.POINTER(OrConvShape)]),
    "or_conv_workspace_floats": (_sz, [C.POINTER(OrConvShape)]),
    "or_conv_forward": (None, [C.POINTER(OrConvShape), _vp, _vp, _vp, _vp]),
    "or_conv_backward": (None, [C.POINTER(OrConvShape), _vp, _vp, _vp, _vp, _vp, _vp]),
    "or_add_bias": (None, [_vp, _vp, _i, _i, _i]),
    "or_bias_grad": (None, [_vp, _vp, _i, _i, _i]),
    "or_bn_mean_var": (None, [_vp, _i, _i, _i, _vp, _vp]),
    "or_bn_roll": (None, [_i, _vp, _vp, _vp, _vp]),
    "or_bn_normalize": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "or_bn_backward": (None, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "or_bn_normalize_roll": (None, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "or_conv_bn_fold": (None, [_i, _i, _vp, _vp, _vp, _vp, _vp]),
    "or_activate": (None, [_vp, _i, _i]),
    "or_gradient": (None, [_vp, _i, _i, _vp]),
    "or_maxpool_out": (_i, [_i, _i, _i, _i]),
    "or_maxpool_forward": (None, [_vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp]),
    "or_maxpool_forward_xy": (None, [_vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp]),
    "or_maxpool_backward": (None, [_vp, _vp, _i, _vp]),
    "or_avgpool_forward": (None, [_vp, _i, _i, _i, _vp]),
    "or_avgpool_backward": (None, [_vp, _i, _i, _i, _vp]),
    "or_softmax_xent_forward": (_f, [_vp, _i, _i, _i, _f, _vp, _vp, _vp, _vp]),
    "or_softmax_backward": (None, [_vp, _i, _vp]),
    "or_dropout_uniform": (_f, [_u64, _u32, _u32, _u32]),
    "or_dropout_forward": (None, [_vp, _i, _f, _u64, _u32, _u32]),
    "or_dropout_backward": (None, [_vp, _i, _f, _u64, _u32, _u32]),
    "or_conv_update": (None, [_i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _f, _f, _f]),
    "or_rand_seed": (None, [C.c_uint]),
    "or_rand_uniform": (_f, [_f, _f]),
    "or_net_create": (_vp, [_i, _i, _i, _i]),
    "or_net_add_conv": (_i, [_vp, _i, _i, _i, _i, _i, _i]),
    "or_net_add_connected": (_i, [_vp, _i, _i, _i]),
    "or_net_add_maxpool": (_i, [_vp, _i, _i, _i]),
    "or_net_add_conv_xy": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i]),
    "or_net_add_maxpool_xy": (_i, [_vp, _i, _i, _i, _i]),
    "or_net_add_avgpool": (_i, [_vp]),
    "or_net_add_dropout": (_i, [_vp, _f]),
    "or_net_add_softmax": (_i, [_vp, _i, _f]),
    "or_net_set_hyper": (None, [_vp, _f, _f, _f]),
    "or_net_set_dropout_seed": (None, [_vp, _u64]),
    "or_lr_rate": (_f, [_i, _f, _u64, _i, _f, _f, _f, _i, _i, _i, _vp, _vp]),
    "or_net_set_policy": (None, [_vp, _i, _i, _f, _f, _f, _i, _i, _i, _vp, _vp]),
    "or_net_set_subdivisions": (None, [_vp, _i]),
    "or_net_rate": (_f, [_vp]),
    "or_net_seen": (_u64, [_vp]),
    "or_net_iteration": (_i, [_vp]),
    "or_net_set_layer_options": (None, [_vp, _i, _i, _i, _f]),
    "or_net_finalize": (_i, [_vp]),
    "or_net_free": (None, [_vp]),
    "or_net_train": (_f, [_vp, _vp, _vp]),
    "or_net_forward_backward": (_f, [_vp, _vp, _vp]),
    "or_net_update": (None, [_vp]),
    "or_net_predict": (None, [_vp, _vp, _vp]),
    "or_net_fuse_conv_batchnorm": (None, [_vp]),
    "or_net_load": (None, [_vp, _vp, _vp]),
    "or_net_layer_forward": (None, [_vp, _i, _i]),
    "or_net_layer_backward": (None, [_vp, _i]),
    "or_net_cost": (_f, [_vp]),
    "or_net_n_layers": (_i, [_vp]),
    "or_net_buffer": (_vp, [_vp, _i, _i, C.POINTER(_sz)]),
    "or_net_layer_info": (None, [_vp, _i, C.POINTER(_i)]),
}

_lib = None


def set_library(path: str):
    """Use another build of the oracle (bench.py's CPU baseline compiles one
    with -march=native on the host it runs on); before the first lib()."""
    global ORACLE_SO
    if _lib is not None and path != ORACLE_SO:
        raise RuntimeError("oracle library already loaded from " + ORACLE_SO)
    ORACLE_SO = path


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} not built (make -C oracle)")
        l = C.CDLL(ORACLE_SO)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def P(a: np.ndarray):
    """ctypes pointer of a contiguous numpy array (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "array must be contiguous"
    return a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- convenience wrappers returning numpy results ---------------------------

def gemm(TA, TB, M, N, K, alpha, A, lda, B, ldb, beta, Cm, ldc):
    Cm = f32(Cm).copy()
    lib().or_gemm(TA, TB, M, N, K, alpha, P(f32(A)), lda, P(f32(B)), ldb, beta, P(Cm), ldc)
    return Cm


def conv_shape(batch, c, h, w, n, size, stride, pad, stride_y=0):
    """stride: the width stride; stride_y 0: the same as stride"""
    return OrConvShape(batch, c, h, w, n, size, stride, pad, stride_y)


def conv_forward(x, w, n, size, stride, pad, stride_y=0):
    B, Cc, H, W = x.shape
    s = conv_shape(B, Cc, H, W, n, size, stride, pad, stride_y)
    oh, ow = lib().or_conv_out_h(C.byref(s)), lib().or_conv_out_w(C.byref(s))
    y = np.zeros((B, n, oh, ow), np.float32)
    ws = np.zeros(max(1, lib().or_conv_workspace_floats(C.byref(s))), np.float32)
    lib().or_conv_forward(C.byref(s), P(f32(x)), P(f32(w)), P(y), P(ws))
    return y


def conv_backward(x, dy, w, size, stride, pad, dw0=None, want_dx=True, stride_y=0):
    B, Cc, H, W = x.shape
    n = dy.shape[1]
    s = conv_shape(B, Cc, H, W, n, size, stride, pad, stride_y)
    dw = np.zeros(w.shape, np.float32) if dw0 is None else f32(dw0).copy()
    dx = np.zeros(x.shape, np.float32) if want_dx else None
    ws = np.zeros(max(1, lib().or_conv_workspace_floats(C.byref(s))), np.float32)
    lib().or_conv_backward(C.byref(s), P(f32(x)), P(f32(dy)), P(f32(w)), P(dw), P(dx), P(ws))
    return dw, dx


def bn_forward(out, scales, biases, rolling_mean=None, rolling_var=None):
    """forwardNormCPU train branch; returns dict of all outputs."""
    out = f32(out).copy()
    B, Cc = out.shape[0], out.shape[1]
    sp = int(np.prod(out.shape[2:]))
    mean = np.zeros(Cc, np.float32)
    var = np.zeros(Cc, np.float32)
    rm = np.zeros(Cc, np.float32) if rolling_mean is None else f32(rolling_mean).copy()
    rv = np.zeros(Cc, np.float32) if rolling_var is None else f32(rolling_var).copy()
    x = np.zeros_like(out)
    xn = np.zeros_like(out)
    lib().or_bn_mean_var(P(out), B, Cc, sp, P(mean), P(var))
    lib().or_bn_roll(Cc, P(mean), P(var), P(rm), P(rv))
    bad = lib().or_bn_normalize(P(out), B, Cc, sp, P(mean), P(var), P(f32(scales)), P(f32(biases)),
                                P(x), P(xn))
    return dict(out=out, mean=mean, var=var, rm=rm, rv=rv, x=x, xn=xn, nan=bad)


def bn_normalize_roll(out, rolling_mean, rolling_var, scales, biases):
    """NormData.normalizeByRoll (inference batch-norm)"""
    out = f32(out).copy()
    B, Cc = out.shape[0], out.shape[1]
    sp = int(np.prod(out.shape[2:]))
    lib().or_bn_normalize_roll(P(out), B, Cc, sp, P(f32(rolling_mean)), P(f32(rolling_var)),
                               P(f32(scales)), P(f32(biases)))
    return out


def conv_bn_fold(weights, biases, scales, rolling_mean, rolling_var):
    """ConvolutionalLayer.fuseConvBatchnorm; returns folded (weights, biases)"""
    w = f32(weights).copy()
    b = f32(biases).copy()
    F = b.shape[0]
    lib().or_conv_bn_fold(F, w.size // F, P(w), P(b), P(f32(scales)), P(f32(rolling_mean)),
                          P(f32(rolling_var)))
    return w, b


def bn_backward(delta, x, xn, mean, var, scales, scale_updates=None):
    d = f32(delta).copy()
    B, Cc = d.shape[0], d.shape[1]
    sp = int(np.prod(d.shape[2:]))
    su = np.zeros(Cc, np.float32) if scale_updates is None else f32(scale_updates).copy()
    md = np.zeros(Cc, np.float32)
    vd = np.zeros(Cc, np.float32)
    lib().or_bn_backward(P(d), B, Cc, sp, P(f32(x)), P(f32(xn)), P(f32(mean)), P(f32(var)),
                         P(f32(scales)), P(su), P(md), P(vd))
    return dict(delta=d, scale_updates=su, mean_delta=md, var_delta=vd)


def activate(x, act):
    y = f32(x).copy()
    lib().or_activate(P(y), y.size, act)
    return y


def gradient(y, act, delta):
    d = f32(delta).copy()
    lib().or_gradient(P(f32(y)), d.size, act, P(d))
    return d


def maxpool_forward(x, size, stride, pad, stride_y=None):
    """stride: the width stride; stride_y (default: stride) the height one"""
    B, Cc, H, W = x.shape
    sy = stride if stride_y is None else stride_y
    oh = lib().or_maxpool_out(H, size, sy, pad)
    ow = lib().or_maxpool_out(W, size, stride, pad)
    out = np.zeros((B, Cc, oh, ow), np.float32)
    idx = np.zeros((B, Cc, oh, ow), np.int32)
    if stride_y is None:
        lib().or_maxpool_forward(P(f32(x)), B, Cc, H, W, size, stride, pad, P(out), P(idx))
    else:
        lib().or_maxpool_forward_xy(P(f32(x)), B, Cc, H, W, size, stride, sy, pad, P(out),
                                    P(idx))
    return out, idx


def maxpool_backward(dout, idx, din0):
    din = f32(din0).copy()
    lib().or_maxpool_backward(P(f32(dout)), P(np.ascontiguousarray(idx, np.int32)), dout.size,
                              P(din))
    return din


def avgpool_forward(x):
    B, Cc = x.shape[:2]
    sp = int(np.prod(x.shape[2:]))
    out = np.zeros((B, Cc), np.float32)
    lib().or_avgpool_forward(P(f32(x)), B, Cc, sp, P(out))
    return out


def avgpool_backward(dout, shape, din0=None):
    B, Cc = shape[:2]
    sp = int(np.prod(shape[2:]))
    din = np.zeros(shape, np.float32) if din0 is None else f32(din0).copy()
    lib().or_avgpool_backward(P(f32(dout)), B, Cc, sp, P(din))
    return din


def softmax_xent(x, truth, groups=1, temperature=1.0):
    x = f32(x)
    B = x.shape[0]
    inputs = x.size // B
    out = np.zeros_like(x)
    delta = np.zeros_like(x)
    err = np.zeros_like(x)
    cost = lib().or_softmax_xent_forward(P(x), B, inputs, groups, temperature,
                                         P(f32(truth)) if truth is not None else None,
                                         P(out), P(delta), P(err))
    return out, delta, err, cost


def dropout_mask_scale(n, p, seed, it, layer):
    ones = np.ones(n, np.float32)
    lib().or_dropout_forward(P(ones), n, p, seed, it, layer)
    return ones


def conv_update(w, dw, b, db, s, ds, batch, lr, mom, decay):
    w, dw, b, db = (f32(a).copy() for a in (w, dw, b, db))
    s = None if s is None else f32(s).copy()
    ds = None if ds is None else f32(ds).copy()
    lib().or_conv_update(w.size, P(w), P(dw), b.size, P(b), P(db), P(s), P(ds), batch, lr, mom,
                         decay)
    return w, dw, b, db, s, ds


class OracleNet:
    """An or_net built layer by layer with the same calls as aetcnn.Network."""

    def __init__(self, batch, h, w, c):
        self.L = lib()
        self.h = self.L.or_net_create(batch, h, w, c)
        self.batch = batch

    def conv(self, filters, size, stride, pad, act, bn, stride_y=None):
        if stride_y is None:
            r = self.L.or_net_add_conv(self.h, filters, size, stride, pad, act, int(bn))
        else:
            r = self.L.or_net_add_conv_xy(self.h, filters, size, stride, stride_y, pad, act,
                                          int(bn))
        assert r >= 0
        return r

    def connected(self, outputs, act, bn):
        r = self.L.or_net_add_connected(self.h, outputs, act, int(bn))
        assert r >= 0
        return r

    def maxpool(self, size, stride, padding, stride_y=None):
        if stride_y is None:
            r = self.L.or_net_add_maxpool(self.h, size, stride, padding)
        else:
            r = self.L.or_net_add_maxpool_xy(self.h, size, stride, stride_y, padding)
        assert r >= 0
        return r

    def avgpool(self):
        return self.L.or_net_add_avgpool(self.h)

    def dropout(self, p):
        return self.L.or_net_add_dropout(self.h, p)

    def softmax(self, groups=1, temperature=1.0):
        return self.L.or_net_add_softmax(self.h, groups, temperature)

    def hyper(self, lr, mom, decay):
        self.L.or_net_set_hyper(self.h, lr, mom, decay)

    def dropout_seed(self, seed):
        self.L.or_net_set_dropout_seed(self.h, seed)

    def policy(self, policy, burn_in=0, power=4.0, gamma=1.0, scale=1.0, step=1,
               max_batches=0, steps=(), scales=()):
        st = np.ascontiguousarray(steps, np.int32)
        sc = np.ascontiguousarray(scales, np.float32)
        assert st.size == sc.size
        self.L.or_net_set_policy(self.h, policy, burn_in, power, gamma, scale, step,
                                 max_batches, st.size, P(st) if st.size else None,
                                 P(sc) if sc.size else None)

    def subdivisions(self, s):
        self.L.or_net_set_subdivisions(self.h, s)

    def rate(self):
        return self.L.or_net_rate(self.h)

    def seen(self):
        return self.L.or_net_seen(self.h)

    def iteration(self):
        return self.L.or_net_iteration(self.h)

    def set_layer_options(self, i, stopbackward=0, onlyforward=0, learning_rate_scale=1.0,
                          **_):
        self.L.or_net_set_layer_options(self.h, i, stopbackward, onlyforward,
                                        learning_rate_scale)

    def finalize(self):
        assert self.L.or_net_finalize(self.h) == 0

    def train(self, x, truth):
        return self.L.or_net_train(self.h, P(f32(x)), P(f32(truth)))

    def forward_backward(self, x, truth):
        return self.L.or_net_forward_backward(self.h, P(f32(x)), P(f32(truth)))

    def update(self):
        self.L.or_net_update(self.h)

    def predict(self, x):
        n = self.n_layers()
        classes = int(np.prod(self.info(n - 1)[1:4]))
        out = np.empty((self.batch, classes), np.float32)
        self.L.or_net_predict(self.h, P(f32(x)), P(out))
        return out

    def fuse_conv_batchnorm(self):
        self.L.or_net_fuse_conv_batchnorm(self.h)

    def load(self, x, truth):
        self.L.or_net_load(self.h, P(f32(x)), P(f32(truth)) if truth is not None else None)

    def layer_forward(self, i, train=1):
        self.L.or_net_layer_forward(self.h, i, train)

    def layer_backward(self, i):
        self.L.or_net_layer_backward(self.h, i)

    def cost(self):
        return self.L.or_net_cost(self.h)

    def n_layers(self):
        return self.L.or_net_n_layers(self.h)

    def buffer(self, layer, which):
        n = _sz()
        p = self.L.or_net_buffer(self.h, layer, which, C.byref(n))
        if not p or n.value == 0:
            return None
        ct = C.c_int if which == 14 else C.c_float
        arr = np.ctypeslib.as_array(C.cast(p, C.POINTER(ct)), shape=(n.value,))
        return arr.copy()

    def set_buffer(self, layer, which, values):
        n = _sz()
        p = self.L.or_net_buffer(self.h, layer, which, C.byref(n))
        v = np.ascontiguousarray(values, np.int32 if which == 14 else np.float32).ravel()
        assert p and v.size == n.value
        C.memmove(p, v.ctypes.data, v.nbytes)

    def info(self, layer):
        a = (C.c_int * 8)()
        self.L.or_net_layer_info(self.h, layer, a)
        return list(a)

    def close(self):
        if self.h:
            self.L.or_net_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# LearningRatePolicy ids (NNetwork.h:29-31)
CONSTANT, STEP, EXP, POLY, STEPS, SIG, RANDOM = range(7)


def lr_rate(policy, lr, batch_num, burn_in=0, power=4.0, gamma=1.0, scale=1.0, step=1,
            max_batches=0, steps=(), scales=()):
    st = np.ascontiguousarray(steps, np.int32)
    sc = np.ascontiguousarray(scales, np.float32)
    return lib().or_lr_rate(policy, lr, batch_num, burn_in, power, gamma, scale, step,
                            max_batches, st.size, P(st) if st.size else None,
                            P(sc) if sc.size else None)
