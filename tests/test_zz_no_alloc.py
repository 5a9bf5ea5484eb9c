"""ach_bn_train_fwd_from_x_noalloc (the allocation-free entry point, partial
sums in a fixed device array) against ach_bn_train_fwd_from_x with a caller
workspace: identical outputs, statistics and rolling statistics, bit for
bit, on two calls in a row -- the second with a smaller input, so it runs on
what the first call left in the shared array -- and a clear refusal of a
shape whose partial sums exceed the array."""
import numpy as np
import pytest

import aetcnn
from aetcnn import DeviceArray as D, check

pytestmark = pytest.mark.gpu


def _bn_pair(gpu, B, Cc, HW, act, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, Cc, HW)).astype(np.float32) * 2 + 0.5
    sc = rng.uniform(0.5, 1.5, Cc).astype(np.float32)
    bi = rng.uniform(-0.2, 0.2, Cc).astype(np.float32)
    rm = rng.uniform(-0.1, 0.1, Cc).astype(np.float32)
    rv = rng.uniform(0.5, 1.5, Cc).astype(np.float32)
    dx, dsc, dbi = D.from_numpy(x), D.from_numpy(sc), D.from_numpy(bi)
    res = []
    for noalloc in (False, True):
        out, m, v = D(x.shape), D(Cc), D(Cc)
        drm, drv = D.from_numpy(rm), D.from_numpy(rv)
        if noalloc:
            check(gpu.ach_bn_train_fwd_from_x_noalloc(dx.ptr, out.ptr, B, Cc, HW, dsc.ptr, dbi.ptr,
                                                      m.ptr, v.ptr, drm.ptr, drv.ptr, act, None),
                  "noalloc")
        else:
            ws = gpu.ach_bn_workspace(B, Cc, HW)
            dws = D(ws // 4 + 64)
            check(gpu.ach_bn_train_fwd_from_x(dx.ptr, out.ptr, B, Cc, HW, dsc.ptr, dbi.ptr, m.ptr,
                                              v.ptr, drm.ptr, drv.ptr, act, dws.ptr, ws, None),
                  "workspace")
        res.append([a.numpy().view(np.uint32) for a in (out, m, v, drm, drv)])
    return res


@pytest.mark.parametrize("first,second", [((128, 256, 256, aetcnn.LEAKY), (16, 64, 100, aetcnn.LINEAR)),
                                          ((64, 4000, 9, aetcnn.RELU), (3, 5, 7, aetcnn.LEAKY))])
def test_bn_noalloc_matches_workspace_variant(gpu, first, second):
    for seed, (B, Cc, HW, act) in enumerate((first, second)):
        ref, got = _bn_pair(gpu, B, Cc, HW, act, seed + 11)
        for name, a, b in zip(("out", "mean", "variance", "rolling_mean", "rolling_variance"),
                              ref, got):
            assert np.array_equal(a, b), (B, Cc, HW, name)


def test_bn_noalloc_rejects_oversized(gpu):
    """partial sums beyond ACH_BN_NOALLOC_SCRATCH_BYTES: ACH_EWORKSPACE, no launch"""
    Cc = 12000
    assert gpu.ach_bn_workspace(1, Cc, 4) > 256 * 1024
    x, out, chan = D((Cc, 4)), D((Cc, 4)), D(Cc)
    rc = gpu.ach_bn_train_fwd_from_x_noalloc(x.ptr, out.ptr, 1, Cc, 4, chan.ptr, chan.ptr,
                                             chan.ptr, chan.ptr, None, None, aetcnn.LINEAR, None)
    assert rc == aetcnn.ACH_EWORKSPACE
    assert b"scratch" in gpu.ach_last_hip_error()
