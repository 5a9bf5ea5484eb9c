"""ctypes bindings for the two in-tree libraries of aet-cnn on MI355X.

``libach.so``    -- the gfx950 HIP kernels behind ``include/aetcnn_ops.h``
``libaetcnn.so`` -- the C host layer (network / layer structs) behind
                    ``include/aetcnn_net.h``

The bindings are plumbing for tests and benchmarks: every computation runs
in the libraries.  Loading fails loudly when a library has not been built;
there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.environ.get("AETCNN_LIB_DIR") or os.path.join(PKG_DIR, "lib")

ACH_OK = 0
ACH_EINVAL = -1
ACH_EWORKSPACE = -2
ACH_EHIP = -3
ACH_EUNSUPPORTED = -4
ACH_ENAN = -5

LOGISTIC, RELU, LINEAR, LEAKY = 0, 1, 3, 7

AN_CONVOLUTIONAL, AN_MAXPOOL, AN_AVGPOOL, AN_DROPOUT, AN_SOFTMAX = 0, 1, 2, 3, 4

# an_policy (the reference's LearningRatePolicy order)
(POLICY_CONSTANT, POLICY_STEP, POLICY_EXP, POLICY_POLY, POLICY_STEPS, POLICY_SIG,
 POLICY_RANDOM) = range(7)

_vp = C.c_void_p
_sz = C.c_size_t
_i = C.c_int
_f = C.c_float
_u64 = C.c_uint64
_u32 = C.c_uint32


class ConvDesc(C.Structure):
    """ach_conv_desc; stride_y 0 (the default) means the same as stride"""
    _fields_ = [("batch", _i), ("c", _i), ("h", _i), ("w", _i), ("n", _i),
                ("size", _i), ("stride", _i), ("pad", _i), ("stride_y", _i)]


class LayerOptions(C.Structure):
    """an_layer_options"""
    _fields_ = [("stopbackward", _i), ("onlyforward", _i), ("dontload", _i),
                ("dontloadscales", _i), ("flipped", _i), ("learning_rate_scale", _f)]


class Validation(C.Structure):
    """an_validation: the result of an_validate_paths"""
    _fields_ = [("images", _i), ("unlabeled", _i), ("topk", _i), ("top1_accuracy", _f),
                ("topk_accuracy", _f)]


class Augment(C.Structure):
    """an_augment: the [net] augmentation keys (defaults: an_augment_defaults)"""
    _fields_ = [("min_crop", _i), ("max_crop", _i), ("angle", _f), ("aspect", _f), ("hue", _f),
                ("saturation", _f), ("exposure", _f), ("flip", _i)]

    @classmethod
    def defaults(cls, net_w, **kw):
        a = cls()
        net_lib().an_augment_defaults(C.byref(a), net_w)
        for k, v in kw.items():
            setattr(a, k, v)
        return a


class FilterJob(C.Structure):
    """ach_filter_job"""
    _fields_ = [("desc", ConvDesc), ("w", _vp), ("wt", _vp), ("wft", _vp)]


# name -> (restype, argtypes)
_OPS = {
    "ach_version": (C.c_char_p, []),
    "ach_device_count": (_i, []),
    "ach_set_device": (_i, [_i]),
    "ach_last_hip_error": (C.c_char_p, []),
    "ach_malloc": (_i, [C.POINTER(_vp), _sz]),
    "ach_free": (_i, [_vp]),
    "ach_host_alloc": (_i, [C.POINTER(_vp), _sz]),
    "ach_host_free": (_i, [_vp]),
    "ach_memcpy_h2d": (_i, [_vp, _vp, _sz, _vp]),
    "ach_memcpy_d2h": (_i, [_vp, _vp, _sz, _vp]),
    "ach_memcpy_h2d_async": (_i, [_vp, _vp, _sz, _vp]),
    "ach_event_sync": (_i, [_vp]),
    "ach_stream_wait_event": (_i, [_vp, _vp]),
    "ach_memcpy_d2d": (_i, [_vp, _vp, _sz, _vp]),
    "ach_stream_create": (_i, [C.POINTER(_vp)]),
    "ach_stream_destroy": (_i, [_vp]),
    "ach_stream_sync": (_i, [_vp]),
    "ach_device_sync": (_i, []),
    "ach_event_create": (_i, [C.POINTER(_vp)]),
    "ach_event_destroy": (_i, [_vp]),
    "ach_event_record": (_i, [_vp, _vp]),
    "ach_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(_f)]),
    "ach_fill": (_i, [_vp, _sz, _f, _vp]),
    "ach_axpy": (_i, [_sz, _f, _vp, _vp, _vp]),
    "ach_scal": (_i, [_sz, _f, _vp, _vp]),
    "ach_gemm": (_i, [_i, _i, _i, _i, _i, _f, _vp, _i, _vp, _i, _f, _vp, _i, _vp]),
    "ach_im2col": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp]),
    "ach_col2im": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp]),
    "ach_conv_out_h": (_i, [C.POINTER(ConvDesc)]),
    "ach_conv_out_w": (_i, [C.POINTER(ConvDesc)]),
    "ach_conv_fwd_workspace": (_sz, [C.POINTER(ConvDesc)]),
    "ach_conv_fwd": (_i, [C.POINTER(ConvDesc), _vp, _vp, _vp, _vp, _sz, _vp]),
    "ach_conv_bwd_data_workspace": (_sz, [C.POINTER(ConvDesc)]),
    "ach_conv_bwd_data": (_i, [C.POINTER(ConvDesc), _vp, _vp, _vp, _vp, _sz, _vp]),
    "ach_conv_bwd_filter_workspace": (_sz, [C.POINTER(ConvDesc)]),
    "ach_conv_bwd_filter": (_i, [C.POINTER(ConvDesc), _vp, _vp, _vp, _vp, _sz, _vp]),
    "ach_conv_bwd_filter_sgd": (_i, [C.POINTER(ConvDesc), _vp, _vp, _vp, _vp, _f, _f, _f, _vp, _sz,
                                    _vp]),
    "ach_conv_bwd_data_reads_w": (_i, [C.POINTER(ConvDesc)]),
    "ach_add_bias": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "ach_bias_grad_workspace": (_sz, [_i, _i, _i]),
    "ach_bias_grad": (_i, [_vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "ach_bias_grad_planes": (_i, [_vp, _vp, _i, _i, _vp]),
    "ach_bn_workspace": (_sz, [_i, _i, _i]),
    "ach_bn_train_fwd": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                              _vp, _sz, _vp]),
    "ach_bn_train_fwd_from_x": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                                     _vp, _sz, _vp]),
    "ach_bn_train_fwd_from_x_noalloc": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _i, _vp]),
    "ach_conv_prepare_filters": (_i, [_i, _vp, _vp]),
    "ach_conv_is_fully_connected": (_i, [C.POINTER(ConvDesc)]),
    "ach_conv_fwd_prepared": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ach_conv_bwd_data_prepared": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ach_conv_fwd_bias_act_prepared": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, _sz, _vp]),
    "ach_bn_infer": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp]),
    "ach_conv_bn_fold": (_i, [_i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ach_bn_bwd": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                        _vp, _sz, _vp]),
    "ach_activate": (_i, [_vp, _sz, _i, _vp]),
    "ach_gradient": (_i, [_vp, _sz, _i, _vp, _vp]),
    "ach_gradient_planes": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "ach_maxpool_out": (_i, [_i, _i, _i, _i]),
    "ach_maxpool_fwd": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp]),
    "ach_maxpool_bwd": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _vp]),
    "ach_maxpool_fwd_xy": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp]),
    "ach_maxpool_bwd_xy": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _vp]),
    "ach_maxpool_bwd_act": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _vp, _i, _vp]),
    "ach_maxpool_bwd_act_planes": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp,
                                        _vp]),
    "ach_maxpool_bwd_act_pooled": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp,
                                        _vp]),
    "ach_maxpool_fwd_dropout": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _f, _u64, _u32,
                                     _u32, _vp]),
    "ach_maxpool_bwd_dropout": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _i, _f, _u64,
                                     _u32, _u32, _vp]),
    "ach_avgpool_fwd": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "ach_avgpool_bwd": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "ach_softmax_workspace": (_sz, [_i, _i]),
    "ach_softmax_xent": (_i, [_vp, _i, _i, _i, _f, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ach_dropout_uniform": (_f, [_u64, _u32, _u32, _u32]),
    "ach_dropout_fwd": (_i, [_vp, _sz, _f, _u64, _u32, _u32, _vp]),
    "ach_dropout_bwd": (_i, [_vp, _sz, _f, _u64, _u32, _u32, _vp]),
    "ach_nan_scan": (_i, [_vp, _i, _vp, _vp]),
    "ach_conv_update": (_i, [_sz, _vp, _vp, _sz, _vp, _vp, _vp, _vp, _i, _f, _f, _f, _vp]),
    "ach_sgd_update": (_i, [_sz, _vp, _vp, _f, _f, _f, _vp]),
}

_NET = {
    "an_rand_seed": (None, [C.c_uint]),
    "an_network_create": (_vp, [_i, _i, _i, _i]),
    "an_add_convolutional": (_i, [_vp, _i, _i, _i, _i, _i, _i]),
    "an_add_connected": (_i, [_vp, _i, _i, _i]),
    "an_add_maxpool": (_i, [_vp, _i, _i, _i]),
    "an_add_convolutional_xy": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i]),
    "an_add_maxpool_xy": (_i, [_vp, _i, _i, _i, _i]),
    "an_add_avgpool": (_i, [_vp]),
    "an_add_dropout": (_i, [_vp, _f]),
    "an_add_softmax": (_i, [_vp, _i, _f]),
    "an_set_hyper": (None, [_vp, _f, _f, _f]),
    "an_set_dropout_seed": (None, [_vp, _u64]),
    "an_set_policy": (_i, [_vp, _i, _i, _f, _f, _f, _i, _i, _i, _vp, _vp]),
    "an_rate": (_f, [_vp, _u64]),
    "an_current_rate": (_f, [_vp]),
    "an_set_subdivisions": (_i, [_vp, _i]),
    "an_finalize": (_i, [_vp]),
    "an_free": (None, [_vp]),
    "an_parse_cfg": (_vp, [C.c_char_p]),
    "an_parse_cfg_unfinalized": (_vp, [C.c_char_p]),
    "an_set_layer_options": (_i, [_vp, _i, C.POINTER(LayerOptions)]),
    "an_get_layer_options": (_i, [_vp, _i, C.POINTER(LayerOptions)]),
    "an_save_weights": (_i, [_vp, C.c_char_p]),
    "an_load_weights": (_i, [_vp, C.c_char_p]),
    "an_stream": (_vp, [_vp]),
    "an_set_input": (_i, [_vp, _vp, _vp]),
    "an_set_input_device": (_i, [_vp, _vp, _vp]),
    "an_train_step": (_i, [_vp]),
    "an_get_loss": (_i, [_vp, C.POINTER(_f)]),
    "an_nan_status": (_i, [_vp, C.POINTER(_i), C.POINTER(_i)]),
    "an_train": (_i, [_vp, _vp, _vp, C.POINTER(_f)]),
    "an_forward": (_i, [_vp, _i]),
    "an_predict": (_i, [_vp, _vp, _vp]),
    "an_fuse_conv_batchnorm": (_i, [_vp]),
    "an_feeder_create_cifar": (_vp, [_vp, _vp, _i, _i, _u64, C.POINTER(Augment), _f]),
    "an_feeder_create_synthetic": (_vp, [_vp, _i, _u64, C.POINTER(Augment)]),
    "an_feeder_create_paths": (_vp, [_vp, C.c_char_p, _vp, _i, _i, _u64, C.POINTER(Augment),
                                     _f]),
    "an_augment_defaults": (None, [C.POINTER(Augment), _i]),
    "an_cfg_augment": (_i, [C.c_char_p, C.POINTER(Augment), C.POINTER(_f)]),
    "an_augment_image": (_i, [_vp, _i, _i, _i, C.POINTER(Augment), _u64, _u64, _i, _vp]),
    "an_image_rotate_crop": (None, [_vp, _i, _i, _i, _f, _f, _i, _i, _f, _f, _f, _vp]),
    "an_image_flip": (None, [_vp, _i, _i, _i]),
    "an_image_distort": (None, [_vp, _i, _i, _f, _f, _f]),
    "an_image_resize": (_i, [_vp, _i, _i, _i, _i, _i, _vp]),
    "an_image_load": (_i, [C.c_char_p, _i, _i, _i, _vp]),
    "an_image_read": (_i, [C.c_char_p, _i, C.POINTER(_i), C.POINTER(_i), C.POINTER(_vp)]),
    "an_image_free": (None, [_vp]),
    "an_image_resize_min_size": (None, [_i, _i, _i, C.POINTER(_i), C.POINTER(_i)]),
    "an_image_crop": (None, [_vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "an_validation_image": (_i, [C.c_char_p, _i, _i, _i, _vp]),
    "an_validate_paths": (_i, [_vp, C.c_char_p, _vp, _i, _i, C.POINTER(Validation)]),
    "an_label_from_path": (_i, [C.c_char_p, _vp, _i]),
    "an_feeder_next": (_i, [_vp]),
    "an_feeder_served": (_u64, [_vp]),
    "an_feeder_sample": (_u64, [_u64, _u64, _i, _i]),
    "an_feeder_free": (None, [_vp]),
    "an_top_k": (None, [_vp, _i, _i, _vp]),
    "an_backward": (_i, [_vp]),
    "an_update": (_i, [_vp]),
    "an_layer_forward": (_i, [_vp, _i, _i]),
    "an_layer_backward": (_i, [_vp, _i]),
    "an_n_layers": (_i, [_vp]),
    "an_get_layer": (_vp, [_vp, _i]),
    "an_layer_shape": (_i, [_vp, _i, C.POINTER(_i)]),
    "an_batch": (_i, [_vp]),
    "an_input": (_vp, [_vp]),
    "an_truth": (_vp, [_vp]),
    "an_classes": (_i, [_vp]),
    "an_seen": (_u64, [_vp]),
    "an_iteration": (_i, [_vp]),
    "an_layer_buffer": (_vp, [_vp, _i, _i, C.POINTER(_sz)]),
    "an_step_conv_gflop": (C.c_double, [_vp]),
}

_libs = {}


def _load(name: str, table: dict) -> C.CDLL:
    if name in _libs:
        return _libs[name]
    path = os.path.join(LIB_DIR, name)
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is not built; run __graft_entry__.build() (make -C aet-cnn_amd)")
    lib = C.CDLL(path)
    for fn, (res, args) in table.items():
        f = getattr(lib, fn)
        f.restype = res
        f.argtypes = args
    _libs[name] = lib
    return lib


def ops() -> C.CDLL:
    """The HIP kernel library (include/aetcnn_ops.h)."""
    return _load("libach.so", _OPS)


def net_lib() -> C.CDLL:
    """The C host network library (include/aetcnn_net.h)."""
    ops()
    return _load("libaetcnn.so", _NET)


def op_symbols():
    return sorted(_OPS)


def net_symbols():
    return sorted(_NET)


class HipError(RuntimeError):
    pass


def check(rc: int, what: str = ""):
    if rc != ACH_OK:
        err = ops().ach_last_hip_error().decode()
        raise HipError(f"{what} failed with code {rc} ({err})")


def gpu_available() -> bool:
    try:
        return ops().ach_device_count() > 0
    except (OSError, RuntimeError):
        return False


class DeviceArray:
    """A device allocation made through ach_malloc, with numpy transfers."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = _vp()
        check(ops().ach_malloc(C.byref(p), max(self.nbytes, 4)), "ach_malloc")
        self.ptr = p.value
        self._owned = True

    @classmethod
    def from_numpy(cls, a: np.ndarray, stream=None) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a, stream)
        return d

    @classmethod
    def wrap(cls, ptr: int, shape, dtype=np.float32) -> "DeviceArray":
        d = cls.__new__(cls)
        d.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        d.dtype = np.dtype(dtype)
        d.nbytes = int(np.prod(d.shape, dtype=np.int64)) * d.dtype.itemsize
        d.ptr = ptr
        d._owned = False
        return d

    def upload(self, a: np.ndarray, stream=None):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        check(ops().ach_memcpy_h2d(self.ptr, a.ctypes.data, self.nbytes, stream), "h2d")

    def numpy(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(ops().ach_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, stream), "d2h")
        return out

    def zero(self, stream=None):
        check(ops().ach_fill(self.ptr, self.nbytes // 4, 0.0, stream), "fill")

    def free(self):
        if self._owned and self.ptr:
            ops().ach_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Network:
    """Thin owner of an ``an_network*`` built layer by layer."""

    def __init__(self, batch: int, h: int, w: int, c: int):
        self.lib = net_lib()
        self.h = self.lib.an_network_create(batch, h, w, c)
        if not self.h:
            raise ValueError("an_network_create failed")
        self.batch = batch

    @classmethod
    def from_cfg(cls, path: str, finalize: bool = True) -> "Network":
        """an_parse_cfg, or with finalize=False an_parse_cfg_unfinalized (host
        only: no device memory is touched until finalize())."""
        lib = net_lib()
        fn = lib.an_parse_cfg if finalize else lib.an_parse_cfg_unfinalized
        h = fn(os.fsencode(path))
        if not h:
            raise ValueError(f"an_parse_cfg({path}) failed")
        n = cls.__new__(cls)
        n.lib = lib
        n.h = h
        n.batch = lib.an_batch(h)
        return n

    def layer_options(self, i: int) -> dict:
        o = LayerOptions()
        check(self.lib.an_get_layer_options(self.h, i, C.byref(o)), "an_get_layer_options")
        return {k: getattr(o, k) for k, _ in LayerOptions._fields_}

    def set_layer_options(self, i: int, **kw):
        """an_set_layer_options (before finalize); unnamed options keep their values"""
        cur = self.layer_options(i)
        cur.update(kw)
        o = LayerOptions(**cur)
        check(self.lib.an_set_layer_options(self.h, i, C.byref(o)), "an_set_layer_options")

    def conv(self, filters, size, stride, pad, activation, bn, stride_y=None):
        """stride is the width stride; stride_y (default: stride) the height one"""
        if stride_y is None:
            r = self.lib.an_add_convolutional(self.h, filters, size, stride, pad, activation,
                                              int(bn))
        else:
            r = self.lib.an_add_convolutional_xy(self.h, filters, size, stride, stride_y, pad,
                                                 activation, int(bn))
        if r < 0:
            raise ValueError(f"an_add_convolutional: {r}")
        return r

    def connected(self, outputs, activation, bn):
        r = self.lib.an_add_connected(self.h, outputs, activation, int(bn))
        if r < 0:
            raise ValueError(f"an_add_connected: {r}")
        return r

    def maxpool(self, size, stride, padding, stride_y=None):
        if stride_y is None:
            r = self.lib.an_add_maxpool(self.h, size, stride, padding)
        else:
            r = self.lib.an_add_maxpool_xy(self.h, size, stride, stride_y, padding)
        if r < 0:
            raise ValueError(f"an_add_maxpool: {r}")
        return r

    def avgpool(self):
        return self.lib.an_add_avgpool(self.h)

    def dropout(self, p):
        r = self.lib.an_add_dropout(self.h, p)
        if r < 0:
            raise ValueError(f"an_add_dropout: {r}")
        return r

    def softmax(self, groups=1, temperature=1.0):
        return self.lib.an_add_softmax(self.h, groups, temperature)

    def hyper(self, lr, momentum, decay):
        self.lib.an_set_hyper(self.h, lr, momentum, decay)

    def dropout_seed(self, seed):
        self.lib.an_set_dropout_seed(self.h, seed)

    def policy(self, policy, burn_in=0, power=4.0, gamma=1.0, scale=1.0, step=1,
               max_batches=0, steps=(), scales=()):
        """NNetwork.getCurrentRate's policy (ids: POLICY_*)."""
        st = np.ascontiguousarray(steps, np.int32)
        sc = np.ascontiguousarray(scales, np.float32)
        if st.size != sc.size:
            raise ValueError("steps and scales need the same length")
        check(self.lib.an_set_policy(self.h, policy, burn_in, power, gamma, scale, step,
                                     max_batches, st.size, st.ctypes.data if st.size else None,
                                     sc.ctypes.data if sc.size else None), "an_set_policy")

    def rate(self, batch_num=None) -> float:
        """getCurrentRate at batch_num (default: the next update's)."""
        if batch_num is None:
            return self.lib.an_current_rate(self.h)
        return self.lib.an_rate(self.h, batch_num)

    def subdivisions(self, s):
        check(self.lib.an_set_subdivisions(self.h, s), "an_set_subdivisions")

    def finalize(self):
        check(self.lib.an_finalize(self.h), "an_finalize")

    @property
    def stream(self):
        return self.lib.an_stream(self.h)

    def n_layers(self):
        return self.lib.an_n_layers(self.h)

    def shape(self, i):
        """[type, out_c, out_h, out_w, c, h, w, batch] of layer i (host only)."""
        a = (_i * 8)()
        check(self.lib.an_layer_shape(self.h, i, a), "an_layer_shape")
        return list(a)

    def set_input(self, x: np.ndarray, truth: Optional[np.ndarray]):
        x = np.ascontiguousarray(x, dtype=np.float32)
        t = None if truth is None else np.ascontiguousarray(truth, dtype=np.float32)
        check(self.lib.an_set_input(self.h, x.ctypes.data, None if t is None else t.ctypes.data),
              "an_set_input")

    def train(self, x: np.ndarray, truth: np.ndarray) -> float:
        x = np.ascontiguousarray(x, dtype=np.float32)
        t = np.ascontiguousarray(truth, dtype=np.float32)
        loss = _f()
        check(self.lib.an_train(self.h, x.ctypes.data, t.ctypes.data, C.byref(loss)), "an_train")
        return loss.value

    def train_step(self):
        check(self.lib.an_train_step(self.h), "an_train_step")

    def predict(self, x: np.ndarray) -> np.ndarray:
        """NNetwork.predict: inference forward, returns [batch][classes]"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty((self.batch, self.lib.an_classes(self.h)), np.float32)
        check(self.lib.an_predict(self.h, x.ctypes.data, out.ctypes.data), "an_predict")
        return out

    def validate(self, list_file: str, labels, topk: int = 1) -> Validation:
        """an_validate_paths (Classifier.validateSingle): top-1 / top-k
        accuracy over an image list with labels from path substrings"""
        arr = _cstrings(labels)
        res = Validation()
        check(self.lib.an_validate_paths(self.h, os.fsencode(list_file), C.cast(arr, _vp),
                                         len(labels), topk, C.byref(res)), "an_validate_paths")
        return res

    def fuse_conv_batchnorm(self):
        """NNetwork.fuseConvBatchnorm: fold the inference BN of every BN conv
        layer into its filters and biases (the layers become plain convs)"""
        check(self.lib.an_fuse_conv_batchnorm(self.h), "an_fuse_conv_batchnorm")

    def loss(self) -> float:
        v = _f()
        check(self.lib.an_get_loss(self.h, C.byref(v)), "an_get_loss")
        return v.value

    def nan_status(self):
        """None while clean, else (layer, what) of the first batch-norm array
        found holding a NaN: what 0 mean, 1 variance, 2 scales, 3 scale
        updates (an_nan_status)."""
        layer, what = _i(), _i()
        rc = self.lib.an_nan_status(self.h, C.byref(layer), C.byref(what))
        if rc < 0:
            check(rc, "an_nan_status")
        return (layer.value, what.value) if rc else None

    def forward(self, train=1):
        check(self.lib.an_forward(self.h, train), "an_forward")

    def backward(self):
        check(self.lib.an_backward(self.h), "an_backward")

    def update(self):
        check(self.lib.an_update(self.h), "an_update")

    def layer_forward(self, i, train=1):
        check(self.lib.an_layer_forward(self.h, i, train), "an_layer_forward")

    def layer_backward(self, i):
        check(self.lib.an_layer_backward(self.h, i), "an_layer_backward")

    def buffer(self, layer: int, which: int) -> Optional[np.ndarray]:
        n = _sz()
        p = self.lib.an_layer_buffer(self.h, layer, which, C.byref(n))
        if not p or n.value == 0:
            return None
        dt = np.int32 if which == 14 else np.float32
        out = np.empty(n.value, dtype=dt)
        check(ops().ach_memcpy_d2h(out.ctypes.data, p, out.nbytes, self.stream), "d2h")
        return out

    def set_buffer(self, layer: int, which: int, values: np.ndarray):
        n = _sz()
        p = self.lib.an_layer_buffer(self.h, layer, which, C.byref(n))
        v = np.ascontiguousarray(values, dtype=np.int32 if which == 14 else np.float32).ravel()
        assert p and v.size == n.value, (layer, which, v.size, n.value)
        check(ops().ach_memcpy_h2d(p, v.ctypes.data, v.nbytes, self.stream), "h2d")

    def conv_gflop(self) -> float:
        return self.lib.an_step_conv_gflop(self.h)

    def save_weights(self, path: str):
        """darknet .weights file (NNetwork.saveWeightsUpto, NNetwork.c:113-146)"""
        check(self.lib.an_save_weights(self.h, os.fsencode(path)), "an_save_weights")

    def load_weights(self, path: str):
        """darknet .weights file (NNetwork.loadWeights, NNetwork.c:64-110)"""
        check(self.lib.an_load_weights(self.h, os.fsencode(path)), "an_load_weights")

    def seen(self) -> int:
        return self.lib.an_seen(self.h)

    def iteration(self) -> int:
        return self.lib.an_iteration(self.h)

    def close(self):
        if self.h:
            self.lib.an_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def image_read(path: str, c: int) -> np.ndarray:
    """an_image_read: a file at its own size as float planes [c][h][w], with
    c channels converted as the reference's stb_image load does"""
    w, h, p = _i(), _i(), _vp()
    lib = net_lib()
    check(lib.an_image_read(os.fsencode(path), c, C.byref(w), C.byref(h), C.byref(p)),
          "an_image_read")
    try:
        arr = np.ctypeslib.as_array(C.cast(p, C.POINTER(_f)), shape=(c, h.value, w.value)).copy()
    finally:
        lib.an_image_free(p)
    return arr


def resize_min_size(W: int, H: int, mn: int):
    """an_image_resize_min_size: (w, h) of NImage.resizeMin"""
    w, h = _i(), _i()
    net_lib().an_image_resize_min_size(W, H, mn, C.byref(w), C.byref(h))
    return w.value, h.value


def image_crop(src: np.ndarray, dx: int, dy: int, w: int, h: int) -> np.ndarray:
    """an_image_crop (NImage.crop) of host planes [c][H][W]"""
    src = np.ascontiguousarray(src, dtype=np.float32)
    c, H, W = src.shape
    dst = np.empty((c, h, w), np.float32)
    net_lib().an_image_crop(src.ctypes.data, W, H, c, dx, dy, w, h, dst.ctypes.data)
    return dst


def image_resize(src: np.ndarray, w: int, h: int) -> np.ndarray:
    """an_image_resize (NImage.resizeImage) of host planes [c][H][W]"""
    src = np.ascontiguousarray(src, dtype=np.float32)
    c, H, W = src.shape
    dst = np.empty((c, h, w), np.float32)
    check(net_lib().an_image_resize(src.ctypes.data, W, H, c, w, h, dst.ctypes.data),
          "an_image_resize")
    return dst


def validation_image(path: str, w: int, h: int, c: int) -> np.ndarray:
    """an_validation_image: read, resize-min, centre crop"""
    dst = np.empty((c, h, w), np.float32)
    check(net_lib().an_validation_image(os.fsencode(path), w, h, c, dst.ctypes.data),
          "an_validation_image")
    return dst


def top_k(a: np.ndarray, k: int) -> np.ndarray:
    """DnnUtils.topK through the C host library: indices of the k largest
    values, largest first (ties as the reference's insertion leaves them)."""
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    idx = np.empty(k, np.int32)
    net_lib().an_top_k(a.ctypes.data, a.size, k, idx.ctypes.data)
    return idx


def _cstrings(items):
    return (C.c_char_p * len(items))(*[os.fsencode(p) for p in items])


class Feeder:
    """Input pipeline (an_feeder_*): worker threads fill pinned host batches,
    next() makes the next one the network's input (copy overlapped with the
    previous step).  Source: an image list file with labels from path
    substrings (paths_list + labels), CIFAR-10 binary batches (cifar_files)
    or synthetic pixels; augment (an Augment) applies the reference's
    training-time augmentation to every image."""

    def __init__(self, net: "Network", cifar_files=None, threads: int = 8, seed: int = 0,
                 augment: Optional[Augment] = None, label_smooth_eps: float = 0.0,
                 paths_list: Optional[str] = None, labels=None):
        self.lib = net_lib()
        self.net = net
        self._augment = augment
        aug = C.byref(augment) if augment is not None else None
        if paths_list:
            self._labels = _cstrings(labels)
            self.h = self.lib.an_feeder_create_paths(net.h, os.fsencode(paths_list),
                                                     C.cast(self._labels, _vp), len(labels),
                                                     threads, seed, aug, label_smooth_eps)
        elif cifar_files:
            arr = _cstrings(cifar_files)
            self._files = arr
            self.h = self.lib.an_feeder_create_cifar(net.h, arr, len(cifar_files), threads, seed,
                                                     aug, label_smooth_eps)
        else:
            self.h = self.lib.an_feeder_create_synthetic(net.h, threads, seed, aug)
        if not self.h:
            raise HipError("an_feeder_create failed (see stderr)")

    def next(self):
        check(self.lib.an_feeder_next(self.h), "an_feeder_next")

    def served(self) -> int:
        return self.lib.an_feeder_served(self.h)

    def close(self):
        if self.h:
            self.lib.an_feeder_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def augment_image(src: np.ndarray, augment: Augment, seed: int, batch_no: int,
                  image: int) -> np.ndarray:
    """an_augment_image on a host image [c][h][w]"""
    src = np.ascontiguousarray(src, dtype=np.float32)
    c, h, w = src.shape
    dst = np.empty_like(src)
    check(net_lib().an_augment_image(src.ctypes.data, w, h, c, C.byref(augment), seed, batch_no,
                                     image, dst.ctypes.data), "an_augment_image")
    return dst


def image_load(path: str, w: int, h: int, c: int) -> np.ndarray:
    """an_image_load: a PNG / JPEG / PPM / PGM file as float planes [c][h][w]"""
    dst = np.empty((c, h, w), np.float32)
    check(net_lib().an_image_load(os.fsencode(path), w, h, c, dst.ctypes.data), "an_image_load")
    return dst


def label_from_path(path: str, labels) -> int:
    arr = _cstrings(labels)
    return net_lib().an_label_from_path(os.fsencode(path), C.cast(arr, _vp), len(labels))
