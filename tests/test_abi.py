"""The C-ABI libraries load and export every declared symbol; host-side
logic (shapes, workspace plans, cfg parsing errors, counter-based RNG,
bench argument handling) checked without a GPU."""
import ctypes as C
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import aetcnn
from aetcnn import configs
from conftest import ROOT

HEADERS = {
    "aetcnn_ops.h": "libach.so",
    "aetcnn_net.h": "libaetcnn.so",
}


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:ach|an)_[A-Za-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_library_exports_every_declared_symbol(header):
    lib = C.CDLL(os.path.join(aetcnn.LIB_DIR, HEADERS[header]))
    names = declared(header)
    assert len(names) > 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_headers():
    ops_decl = set(declared("aetcnn_ops.h"))
    net_decl = set(declared("aetcnn_net.h"))
    assert ops_decl <= set(aetcnn.op_symbols()), ops_decl - set(aetcnn.op_symbols())
    assert net_decl <= set(aetcnn.net_symbols()), net_decl - set(aetcnn.net_symbols())
    aetcnn.ops()
    aetcnn.net_lib()


def test_conv_shape_and_workspace_queries():
    ops = aetcnn.ops()
    d = aetcnn.ConvDesc(128, 3, 227, 227, 96, 11, 4, 0)
    assert ops.ach_conv_out_h(C.byref(d)) == 55 and ops.ach_conv_out_w(C.byref(d)) == 55
    assert ops.ach_conv_fwd_workspace(C.byref(d)) >= 96 * 3 * 121 * 4
    bad = aetcnn.ConvDesc(1, 3, 2, 2, 4, 5, 1, 0)  # kernel larger than padded input
    assert ops.ach_conv_out_h(C.byref(bad)) == -1
    # split-K partial buffers appear only when the tile grid is small, and
    # not for a forward whose two K slices share one workgroup (256 tiles)
    small = aetcnn.ConvDesc(128, 512, 8, 8, 512, 3, 1, 1)
    big = aetcnn.ConvDesc(128, 128, 32, 32, 128, 3, 1, 1)
    filt = 512 * 512 * 9 * 4
    assert ops.ach_conv_bwd_data_workspace(C.byref(small)) > filt + 512
    assert filt <= ops.ach_conv_fwd_workspace(C.byref(small)) < filt + 512
    assert ops.ach_conv_fwd_workspace(C.byref(big)) < 128 * 128 * 9 * 4 + 512
    fewer = aetcnn.ConvDesc(64, 512, 8, 8, 512, 3, 1, 1)  # 128 tiles: split in four
    assert ops.ach_conv_fwd_workspace(C.byref(fewer)) > filt + 512
    # an odd k-tile count (34 channels: 17 tiles) splits into 9 + 8 tiles,
    # which keep separate workgroups and partial sums
    odd = aetcnn.ConvDesc(2, 34, 8, 8, 128, 3, 1, 1)
    even = aetcnn.ConvDesc(2, 36, 8, 8, 128, 3, 1, 1)
    assert ops.ach_conv_fwd_workspace(C.byref(odd)) >= 34 * 128 * 9 * 4 + 2 * 128 * 2 * 64 * 4
    assert ops.ach_conv_fwd_workspace(C.byref(even)) < 36 * 128 * 9 * 4 + 512
    assert ops.ach_conv_bwd_filter_workspace(C.byref(big)) > 0
    assert ops.ach_maxpool_out(32, 2, 2, 1) == 16  # darknet default padding = size-1
    assert ops.ach_maxpool_out(55, 3, 2, 0) == 27
    # fully connected geometry: a kernel covering the unpadded input, or 1x1 on 1x1
    fc = lambda *a: ops.ach_conv_is_fully_connected(C.byref(aetcnn.ConvDesc(*a)))
    assert fc(128, 256, 6, 6, 4096, 6, 1, 0) == 1
    assert fc(128, 4096, 1, 1, 4096, 1, 1, 0) == 1
    assert fc(128, 256, 6, 6, 4096, 6, 1, 1) == 0   # padded
    assert fc(128, 512, 8, 8, 10, 1, 1, 0) == 0     # 1x1 on an 8x8 plane
    assert fc(128, 256, 7, 6, 4096, 6, 1, 0) == 0   # kernel covers 6 of 7 rows


def test_dropout_generator_matches_oracle(oracle):
    ops = aetcnn.ops()
    for args in [(1, 0, 0, 0), (0x5EED, 7, 3, 12345), (2**63, 2**31, 17, 2**32 - 1)]:
        assert ops.ach_dropout_uniform(*args) == oracle.lib().or_dropout_uniform(*args)


def test_network_shapes_match_oracle(oracle):
    for name, batch in [("tiny", 4), ("darknet", 2), ("alexnet", 2)]:
        net = aetcnn.Network(*configs.dims(name, batch))
        configs.build(net, name)
        onet = oracle.OracleNet(*configs.dims(name, batch))
        configs.build(onet, name)
        assert net.n_layers() == onet.n_layers()
        for i in range(net.n_layers()):
            assert net.shape(i) == onet.info(i), (name, i)
        net.close()
        onet.close()
    # AlexNet-style with padding=0 pools: 55 -> 27 -> 13 -> 6, FC input 9216
    net = aetcnn.Network(*configs.dims("alexnet", 1))
    configs.build(net, "alexnet")
    assert net.shape(7)[1:4] == [256, 6, 6]
    net.close()


def test_layer_constructors_reject_bad_shapes():
    lib = aetcnn.net_lib()
    h = lib.an_network_create(2, 4, 4, 3)
    assert lib.an_add_convolutional(h, 8, 7, 1, 0, aetcnn.LEAKY, 1) < 0   # 7x7 on 4x4
    assert lib.an_add_convolutional(h, 8, 3, 1, 1, 5, 1) == aetcnn.ACH_EUNSUPPORTED
    assert lib.an_add_dropout(h, 1.5) < 0
    assert lib.an_add_convolutional(h, 8, 3, 1, 1, aetcnn.LEAKY, 1) == 0
    assert lib.an_add_softmax(h, 3, 1.0) < 0                              # 128 % 3 != 0
    lib.an_free(h)
    assert lib.an_network_create(0, 4, 4, 3) is None


def test_unequal_strides_shapes_and_errors():
    """Width / height strides on the host: output sizes
    (ConvolutionalLayer.c:337-344, MaxPoolLayer.c:40-41), the per-image
    column buffer as every workspace, and the builders' argument checks."""
    ops = aetcnn.ops()
    d = aetcnn.ConvDesc(4, 5, 13, 10, 6, 3, 2, 1, 3)  # stride_x 2, stride_y 3
    oh, ow = (13 + 2 - 3) // 3 + 1, (10 + 2 - 3) // 2 + 1
    assert (ops.ach_conv_out_h(C.byref(d)), ops.ach_conv_out_w(C.byref(d))) == (oh, ow)
    col = 5 * 9 * oh * ow * 4
    for q in (ops.ach_conv_fwd_workspace, ops.ach_conv_bwd_data_workspace,
              ops.ach_conv_bwd_filter_workspace):
        assert q(C.byref(d)) == col
    assert ops.ach_conv_bwd_data_reads_w(C.byref(d)) == 1
    assert ops.ach_conv_is_fully_connected(C.byref(d)) == 0
    # stride_y 0 or equal to stride: the square-stride descriptor, unchanged
    for sy in (0, 2):
        e = aetcnn.ConvDesc(4, 5, 13, 10, 6, 3, 2, 1, sy)
        sq = aetcnn.ConvDesc(4, 5, 13, 10, 6, 3, 2, 1)
        assert ops.ach_conv_out_h(C.byref(e)) == (13 + 2 - 3) // 2 + 1
        assert ops.ach_conv_fwd_workspace(C.byref(e)) == ops.ach_conv_fwd_workspace(C.byref(sq))
    assert ops.ach_conv_out_h(C.byref(aetcnn.ConvDesc(4, 5, 13, 10, 6, 3, 2, 1, -1))) == -1
    lib = aetcnn.net_lib()
    h = lib.an_network_create(2, 12, 20, 3)
    assert lib.an_add_convolutional_xy(h, 8, 3, 0, 1, 1, aetcnn.LEAKY, 1) == aetcnn.ACH_EINVAL
    assert lib.an_add_convolutional_xy(h, 8, 3, 2, 0, 1, aetcnn.LEAKY, 1) == aetcnn.ACH_EINVAL
    assert lib.an_add_convolutional_xy(h, 8, 3, 2, 1, 1, aetcnn.LEAKY, 1) == 0   # 12 x 10
    assert lib.an_add_maxpool_xy(h, 2, 1, 0, 1) == aetcnn.ACH_EINVAL
    assert lib.an_add_maxpool_xy(h, 3, 1, 2, 2) == 1                           # 6 x 10
    shape = (C.c_int * 8)()
    assert lib.an_layer_shape(h, 0, shape) == 0 and list(shape)[1:4] == [8, 12, 10]
    assert lib.an_layer_shape(h, 1, shape) == 0 and list(shape)[1:4] == [8, 6, 10]
    lib.an_free(h)


def test_cfg_parser_error_paths(tmp_path):
    lib = aetcnn.net_lib()
    assert lib.an_parse_cfg(str(tmp_path / "missing.cfg").encode()) is None
    p = tmp_path / "nonet.cfg"
    p.write_text("[convolutional]\nfilters=4\n")
    assert lib.an_parse_cfg(str(p).encode()) is None
    p.write_text("[net]\nbatch=2\nheight=8\nwidth=8\nchannels=3\n[yolo]\n")
    assert lib.an_parse_cfg(str(p).encode()) is None
    p.write_text("[net]\nbatch=2\nheight=8\nwidth=8\nchannels=3\n"
                 "[convolutional]\nfilters=4\nsize=3\nxnor=1\n")
    assert lib.an_parse_cfg(str(p).encode()) is None


def test_cfg_files_describe_the_configs():
    """The shipped .cfg files parse into the same layer sequence as the
    programmatic configs (checked through the darknet key semantics)."""
    for name in ("tiny", "darknet", "alexnet"):
        text = open(os.path.join(ROOT, "aet-cnn_amd", "cfg", f"{name}.cfg")).read()
        sections = re.findall(r"^\[(\w+)\]", text, flags=re.M)
        kinds = [l[0] for l in configs.CONFIGS[name]["layers"]]
        assert sections[0] == "net"
        assert [s.replace("convolutional", "conv") for s in sections[1:]] == kinds, name


def test_step_flops_match_survey():
    # conv GEMM work per step: config 3 ~813.8 GF, config 0 ~1.15 GF, config 4 ~845 GF
    assert abs(configs.step_gflop("darknet") - 813.8) < 1.0
    assert abs(configs.step_gflop("tiny") - 1.15) < 0.05
    assert abs(configs.step_gflop("alexnet") - 845) / 845 < 0.02


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_finalize_without_device_fails_loudly():
    if aetcnn.gpu_available():
        pytest.skip("a device is present")
    net = aetcnn.Network(2, 8, 8, 3)
    net.conv(4, 3, 1, 1, aetcnn.LEAKY, 1)
    net.softmax()
    with pytest.raises(aetcnn.HipError):
        net.finalize()


def test_top_k_matches_reference_ranking():
    """an_top_k (DnnUtils.topK, DnnUtils.c:463-477): the k largest, largest
    first.  Distinct values: exactly the descending order.  With ties the
    values are still the k largest, non-increasing, with distinct indices
    (their relative order is the reference's insertion order)."""
    rng = np.random.default_rng(4)
    for n, k in [(10, 1), (10, 5), (1000, 5), (7, 7)]:
        a = rng.standard_normal(n).astype(np.float32)
        assert list(aetcnn.top_k(a, k)) == list(np.argsort(-a, kind="stable")[:k]), (n, k)
        t = rng.integers(0, 6, n).astype(np.float32)  # many ties
        idx = aetcnn.top_k(t, k)
        assert len(set(idx.tolist())) == k and idx.min() >= 0
        assert np.array_equal(t[idx], np.sort(t)[::-1][:k]), (n, k)


def test_argument_validation_without_device():
    """Zero-size work returns ACH_OK before touching the device; malformed
    shapes, missing buffers and short workspaces are rejected with codes."""
    ops = aetcnn.ops()
    OK, EINVAL, EWS = 0, aetcnn.ACH_EINVAL, -2
    assert ops.ach_activate(None, 0, aetcnn.LEAKY, None) == OK
    assert ops.ach_activate(None, 0, aetcnn.LINEAR, None) == OK
    assert ops.ach_gradient(None, 0, aetcnn.LEAKY, None, None) == OK
    assert ops.ach_activate(None, 16, aetcnn.LEAKY, None) == EINVAL
    assert ops.ach_dropout_fwd(None, 0, 0.5, 1, 0, 0, None) == OK
    assert ops.ach_dropout_fwd(C.c_void_p(64).value, 8, 1.5, 1, 0, 0, None) == EINVAL
    assert ops.ach_gemm(0, 0, 0, 5, 5, 1.0, None, 5, None, 5, 0.0, C.c_void_p(64).value, 5,
                        None) == OK
    bad = aetcnn.ConvDesc(2, 3, 4, 4, 8, 7, 1, 0)  # 7x7 kernel on a 4x4 image
    fake = C.c_void_p(256).value
    assert ops.ach_conv_fwd(C.byref(bad), fake, fake, fake, fake, 1 << 20, None) == EINVAL
    assert ops.ach_conv_fwd(C.byref(aetcnn.ConvDesc(2, 3, 8, 8, 8, 3, 1, 1)), None, fake, fake,
                            fake, 1 << 20, None) == EINVAL
    small = aetcnn.ConvDesc(128, 512, 8, 8, 512, 3, 1, 1)  # needs split-K scratch
    assert ops.ach_conv_fwd(C.byref(small), fake, fake, fake, fake, 16, None) == EWS
    assert ops.ach_bn_train_fwd_from_x(fake, fake, 0, 4, 16, fake, fake, fake, fake, None, None,
                                       aetcnn.LINEAR, fake, 1 << 20, None) == EINVAL
    other = C.c_void_p(512).value
    assert ops.ach_bn_train_fwd_from_x(fake, fake, 2, 4, 16, fake, fake, fake, fake, None, None,
                                       aetcnn.LINEAR, fake, 1 << 20, None) == EINVAL  # x == out
    assert ops.ach_bn_train_fwd_from_x(fake, other, 2, 4, 16, fake, fake, fake, fake, None, None,
                                       aetcnn.LINEAR, fake, 0, None) == EWS
    assert ops.ach_maxpool_fwd(fake, 1, 1, 4, 4, 0, 2, 0, fake, None, None) == EINVAL
    assert ops.ach_bias_grad(fake, fake, 2, 4, 16, None, 0, None) == EWS
    assert ops.ach_conv_prepare_filters(0, None, None) == OK
    # im2col / col2im take the reference's dilation arguments (>= 1)
    for f in (ops.ach_im2col, ops.ach_col2im):
        assert f(fake, 3, 8, 8, 3, 3, 1, 1, 1, 1, 1, 0, fake, None) == EINVAL
        assert f(fake, 3, 8, 8, 3, 3, 1, 1, 1, 1, 5, 1, fake, None) == EINVAL  # window > input
    assert ops.ach_conv_bwd_data_prepared(C.byref(aetcnn.ConvDesc(2, 3, 9, 9, 8, 3, 2, 1)),
                                          fake, fake, fake, fake, fake, 1 << 20, None) == -4
    # operands at or above 2 GiB (32-bit buffer offsets): refused, never launched
    huge = aetcnn.ConvDesc(1024, 256, 64, 64, 8, 3, 1, 1)  # x = 4 GiB
    for f in (ops.ach_conv_fwd, ops.ach_conv_bwd_data):
        assert f(C.byref(huge), fake, fake, fake, fake, 1 << 40, None) == -4
    assert ops.ach_conv_bwd_filter(C.byref(huge), fake, fake, fake, fake, 1 << 40, None) == -4
    assert ops.ach_conv_fwd_bias_act_prepared(C.byref(huge), fake, fake, None, aetcnn.LEAKY,
                                              fake, fake, 1 << 40, None) == -4
    # the fused forward refuses activations it does not implement
    assert ops.ach_conv_fwd_bias_act_prepared(C.byref(aetcnn.ConvDesc(2, 3, 8, 8, 8, 3, 1, 1)),
                                              fake, fake, None, 2, fake, fake, 1 << 20,
                                              None) == -4
