"""The benchmark networks (3 and 4) as layer lists.

``build(builder, name)`` calls ``conv / maxpool / avgpool / dropout / softmax
/ hyper`` on any object with those methods, so the same description drives
the HIP network (aetcnn.Network) and, in tests, the CPU oracle network.
The .cfg files under ``aet-cnn_amd/cfg/`` describe the same networks in the
reference's darknet format.
"""
from __future__ import annotations

import numpy as np

LOGISTIC, RELU, LINEAR, LEAKY = 0, 1, 3, 7

# name -> dict(batch, h, w, c, classes, lr, momentum, decay, layers)
# layer tuples: ("conv", filters, size, stride, pad, activation, bn[, stride_y])
#               ("connected", outputs, activation, bn)
#               ("maxpool", size, stride, padding[, stride_y])   ("avgpool",)
# (stride is the width stride; stride_y, when given, the height stride)
#               ("dropout", p)   ("softmax",)
CONFIGS = {
    # config 0: tiny CNN
    "tiny": dict(batch=128, h=32, w=32, c=3, classes=10, lr=0.01, momentum=0.9, decay=5e-4,
                 layers=[("conv", 16, 3, 1, 1, LEAKY, 1), ("maxpool", 2, 2, 1),
                         ("conv", 32, 3, 1, 1, LEAKY, 1), ("maxpool", 2, 2, 1),
                         ("conv", 10, 1, 1, 0, LINEAR, 0), ("avgpool",), ("softmax",)]),
    # config 3: darknet-style 32x32 classifier (cifar_small-like)
    "darknet": dict(batch=128, h=32, w=32, c=3, classes=10, lr=0.1, momentum=0.9, decay=5e-4,
                    layers=[("conv", 128, 3, 1, 1, LEAKY, 1)] * 3 +
                    [("maxpool", 2, 2, 1), ("dropout", 0.5)] +
                    [("conv", 256, 3, 1, 1, LEAKY, 1)] * 3 +
                    [("maxpool", 2, 2, 1), ("dropout", 0.5)] +
                    [("conv", 512, 3, 1, 1, LEAKY, 1)] * 3 +
                    [("dropout", 0.5), ("conv", 10, 1, 1, 0, LINEAR, 0), ("avgpool",),
                     ("softmax",)]),
    # fully connected layers on a non-square input (test net, not a benchmark
    # config): conv -> maxpool -> connected+BN -> dropout -> connected -> softmax
    "fcnet": dict(batch=16, h=6, w=10, c=3, classes=10, lr=0.05, momentum=0.9, decay=5e-4,
                  layers=[("conv", 8, 3, 1, 1, LEAKY, 1), ("maxpool", 2, 2, 1),
                          ("connected", 24, LEAKY, 1), ("dropout", 0.5),
                          ("connected", 10, LINEAR, 0), ("softmax",)]),
    # unequal width / height strides (test net, not a benchmark config): a
    # conv entry's optional 8th field and a maxpool entry's optional 5th are
    # the height stride (the 4th / 3rd being the width stride).  BN conv
    # 2x1, pool 1x2, a plain conv (128-position planes) under a 2x1 pool, a
    # 1x2 conv and a 2x1 1x1 conv.
    "stridenet": dict(batch=16, h=16, w=32, c=3, classes=10, lr=0.05, momentum=0.9,
                      decay=5e-4,
                      layers=[("conv", 8, 3, 2, 1, LEAKY, 1, 1), ("maxpool", 2, 1, 1, 2),
                              ("conv", 12, 3, 1, 1, RELU, 0), ("maxpool", 2, 2, 0, 1),
                              ("conv", 16, 3, 1, 1, LEAKY, 0, 2),
                              ("conv", 10, 1, 2, 0, LINEAR, 0, 1), ("avgpool",),
                              ("softmax",)]),
    # config 4: AlexNet-style; FC layers expressed as convolutions
    "alexnet": dict(batch=128, h=227, w=227, c=3, classes=1000, lr=0.01, momentum=0.9,
                    decay=5e-4,
                    layers=[("conv", 96, 11, 4, 0, RELU, 0), ("maxpool", 3, 2, 0),
                            ("conv", 256, 5, 1, 2, RELU, 0), ("maxpool", 3, 2, 0),
                            ("conv", 384, 3, 1, 1, RELU, 0), ("conv", 384, 3, 1, 1, RELU, 0),
                            ("conv", 256, 3, 1, 1, RELU, 0), ("maxpool", 3, 2, 0),
                            ("conv", 4096, 6, 1, 0, RELU, 0), ("dropout", 0.5),
                            ("conv", 4096, 1, 1, 0, RELU, 0), ("dropout", 0.5),
                            ("conv", 1000, 1, 1, 0, LINEAR, 0), ("softmax",)]),
}


def build(builder, name: str, batch: int | None = None):
    cfg = CONFIGS[name]
    for layer in cfg["layers"]:
        kind = layer[0]
        if kind == "conv":
            builder.conv(*layer[1:])
        elif kind == "connected":
            builder.connected(*layer[1:])
        elif kind == "maxpool":
            builder.maxpool(*layer[1:])
        elif kind == "avgpool":
            builder.avgpool()
        elif kind == "dropout":
            builder.dropout(layer[1])
        elif kind == "softmax":
            builder.softmax()
        else:
            raise ValueError(kind)
    builder.hyper(cfg["lr"], cfg["momentum"], cfg["decay"])
    return builder


def dims(name: str, batch: int | None = None):
    cfg = CONFIGS[name]
    return (batch or cfg["batch"], cfg["h"], cfg["w"], cfg["c"])


def synthetic_batch(name: str, seed: int, batch: int | None = None):
    """Pixels uniform [0,1), labels uniform over the classes -> one-hot."""
    cfg = CONFIGS[name]
    B = batch or cfg["batch"]
    rng = np.random.default_rng(seed)
    x = rng.random((B, cfg["c"], cfg["h"], cfg["w"]), dtype=np.float32)
    labels = rng.integers(0, cfg["classes"], B)
    truth = np.zeros((B, cfg["classes"]), np.float32)
    truth[np.arange(B), labels] = 1.0
    return x, truth, labels


def step_gflop(name: str, batch: int | None = None) -> float:
    """Conv GEMM GFLOP of one training step (fwd + wgrad + dgrad; layer 0
    has no input gradient)."""
    cfg = CONFIGS[name]
    B = batch or cfg["batch"]
    h, w, c = cfg["h"], cfg["w"], cfg["c"]
    tot, first = 0.0, True
    for layer in cfg["layers"]:
        if layer[0] == "conv":
            f, k, s, p = layer[1:5]
            sy = layer[7] if len(layer) > 7 else s
            oh, ow = (h + 2 * p - k) // sy + 1, (w + 2 * p - k) // s + 1
            tot += 2.0 * B * f * oh * ow * c * k * k * (2 if first else 3)
            first = False
            h, w, c = oh, ow, f
        elif layer[0] == "maxpool":
            k, s, p = layer[1:4]
            sy = layer[4] if len(layer) > 4 else s
            h, w = (h + p - k) // sy + 1, (w + p - k) // s + 1
        elif layer[0] == "avgpool":
            h = w = 1
    return tot / 1e9
