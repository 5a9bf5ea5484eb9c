#!/usr/bin/env python3
"""Writes the oracle's training-loss curves for BASELINE configs 3 (darknet)
and 4 (AlexNet) at batch 128 -- the fixtures the GPU loss-curve tests
compare against.

The oracle is the plain-C restatement of the reference CPU training path
(oracle/oracle.c), run with its row-parallel GEMM (bit-identical to the
serial order).  Every step trains on a fresh synthetic batch
(configs.synthetic_batch(name, BATCH_SEED + step)); weights come from the
reference's rand() sequence after srand(WEIGHT_SEED); dropout masks from the
counter-based generator with DROPOUT_SEED.

usage: python tests/golden/make_loss_curves.py [darknet|alexnet ...] [--steps N]
"""
import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "aet-cnn_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

from aetcnn import configs  # noqa: E402
import oracle_lib  # noqa: E402

WEIGHT_SEED = 1
DROPOUT_SEED = 0x5EED
BATCH_SEED = 1000


def curve(name, steps, batch):
    L = oracle_lib.lib()
    L.or_set_gemm_parallel(1)
    L.or_rand_seed(WEIGHT_SEED)
    B, h, w, c = configs.dims(name, batch)
    onet = oracle_lib.OracleNet(B, h, w, c)
    configs.build(onet, name)
    onet.dropout_seed(DROPOUT_SEED)
    onet.finalize()
    losses = []
    t0 = time.time()
    for step in range(steps):
        x, truth, _ = configs.synthetic_batch(name, BATCH_SEED + step, B)
        losses.append(float(onet.train(x, truth)))
        print(f"{name} step {step} loss {losses[-1]:.6f} ({time.time() - t0:.0f} s)", flush=True)
    onet.close()
    return dict(config=name, batch=B, steps=steps, weight_seed=WEIGHT_SEED,
                dropout_seed=DROPOUT_SEED, batch_seed=BATCH_SEED, losses=losses,
                generator="tests/golden/make_loss_curves.py (oracle, row-parallel GEMM)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("configs", nargs="*", default=["darknet", "alexnet"])
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--batch", type=int, default=128)
    a = ap.parse_args()
    for name in a.configs:
        d = curve(name, a.steps, a.batch)
        out = os.path.join(HERE, f"{name}_b{d['batch']}_loss{a.steps}.json")
        with open(out, "w") as f:
            json.dump(d, f, indent=1)
        print("wrote", out)


if __name__ == "__main__":
    main()
