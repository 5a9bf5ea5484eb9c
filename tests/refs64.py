"""Float64 brute-force references shared by the CPU oracle pins and the
GPU parity tests (independent of both implementations)."""
import numpy as np


# s is the width stride and sy the height stride (default: s)
def conv_ref(x, w, s, p, sy=None):
    sy = s if sy is None else sy
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    B, Cc, H, W = x.shape
    F, _, k, _ = w.shape
    OH, OW = (H + 2 * p - k) // sy + 1, (W + 2 * p - k) // s + 1
    xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p)))
    out = np.zeros((B, F, OH, OW))
    for ki in range(k):
        for kj in range(k):
            patch = xp[:, :, ki:ki + sy * (OH - 1) + 1:sy, kj:kj + s * (OW - 1) + 1:s]
            out += np.einsum("bchw,fc->bfhw", patch, w[:, :, ki, kj])
    return out


def dgrad_ref(dy, w, xshape, s, p, sy=None):
    sy = s if sy is None else sy
    dy = dy.astype(np.float64)
    w = w.astype(np.float64)
    B, Cc, H, W = xshape
    F, _, k, _ = w.shape
    OH, OW = dy.shape[2:]
    dxp = np.zeros((B, Cc, H + 2 * p, W + 2 * p))
    for ki in range(k):
        for kj in range(k):
            dxp[:, :, ki:ki + sy * (OH - 1) + 1:sy, kj:kj + s * (OW - 1) + 1:s] += \
                np.einsum("bfhw,fc->bchw", dy, w[:, :, ki, kj])
    return dxp[:, :, p:p + H, p:p + W]


def wgrad_ref(x, dy, k, s, p, sy=None):
    sy = s if sy is None else sy
    x = x.astype(np.float64)
    dy = dy.astype(np.float64)
    B, Cc, H, W = x.shape
    F, OH, OW = dy.shape[1:]
    xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p)))
    dw = np.zeros((F, Cc, k, k))
    for ki in range(k):
        for kj in range(k):
            patch = xp[:, :, ki:ki + sy * (OH - 1) + 1:sy, kj:kj + s * (OW - 1) + 1:s]
            dw[:, :, ki, kj] = np.einsum("bfhw,bchw->fc", dy, patch)
    return dw


def bn_backward_ref(delta, y, x, mean, var, scales, act_leaky=True):
    """Batch-norm backward in float64 with the reference CPU path's
    semantics (NLayer.c:246-278, DeltaData.c:23-80): leaky gradient taken on
    the layer output y, eps 1e-5 inside the square root, /N terms, the
    forward's unbiased variance.  Returns (delta', dgamma)."""
    d = delta.astype(np.float64)
    if act_leaky:
        d = d * np.where(y > 0, 1.0, np.float64(np.float32(0.1)))
    m = mean.astype(np.float64)[None, :, None, None]
    v = var.astype(np.float64)[None, :, None, None]
    g = scales.astype(np.float64)[None, :, None, None]
    xc = x.astype(np.float64) - m
    N = d.shape[0] * d.shape[2] * d.shape[3]
    xn = xc / (np.sqrt(v) + 1e-6)
    dgamma = (d * xn).sum(axis=(0, 2, 3))
    dyh = d * g
    s = np.sqrt(v + 1e-5)
    mean_delta = -dyh.sum(axis=(0, 2, 3), keepdims=True) / s
    var_delta = (dyh * xc).sum(axis=(0, 2, 3), keepdims=True) * -0.5 * (v + 1e-5) ** -1.5
    out = dyh / s + var_delta * 2 * xc / N + mean_delta / N
    return out, dgamma
