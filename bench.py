#!/usr/bin/env python3
"""Benchmark: aet-cnn CNN training step on one MI355X.

Headline (BASELINE.json metric): train images/s of the darknet-style 32x32
classifier (config 3: 9x conv3x3+BN+leaky, 1x1 conv, pools, dropout,
softmax) at batch 128, fp32, one full SGD step per iteration, plus the conv
fwd+dgrad+wgrad TFLOP/s of the config-1 layer sweep.  Inputs are synthetic
(seeded uniform pixels and labels) and resident in HBM before timing.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "aet-cnn_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

MFMA_FP32_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0

SWEEP = [  # config 1: (C_in, C_out, H, k, pad)
    (3, 128, 32, 3, 1), (128, 128, 32, 3, 1), (128, 256, 16, 3, 1), (256, 256, 16, 3, 1),
    (256, 512, 8, 3, 1), (512, 512, 8, 3, 1), (512, 10, 8, 1, 0),
]
ROOFLINE_SHAPE = (256, 256, 16, 3, 1)  # dominant kernel probe: conv fwd GEMM
# HBM bytes per probe call (filter transpose + split-K GEMM + split-K
# reduction), from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs scaled by a
# 256 MiB copy dispatch (profiles/conv_fwd_gemm_darknet_b128.md):
# GEMM 53.7 MB read + 67.1 MB written, reduction 67.1 + 33.6 MB,
# transpose 2.4 + 2.4 MB.
ROOFLINE_TRAFFIC_BYTES = 226.2e6


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def train_phase(aetcnn, configs, name, steps, warmup, batch):
    lib = aetcnn.net_lib()
    lib.an_rand_seed(1)
    B, h, w, c = configs.dims(name, batch)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, name)
    net.finalize()
    x, truth, _ = configs.synthetic_batch(name, 1234, B)
    net.set_input(x, truth)  # resident in HBM from here on
    ops = aetcnn.ops()
    for i in range(warmup):
        net.train_step()
    first_loss = net.loss() if warmup else float("nan")
    ops.ach_device_sync()
    ev0, ev1 = C.c_void_p(), C.c_void_p()
    ops.ach_event_create(C.byref(ev0))
    ops.ach_event_create(C.byref(ev1))
    t0 = time.perf_counter()
    ops.ach_event_record(ev0, net.stream)
    for i in range(steps):
        net.train_step()
    ops.ach_event_record(ev1, net.stream)
    aetcnn.check(ops.ach_device_sync(), "sync")
    t1 = time.perf_counter()
    ms = C.c_float()
    ops.ach_event_elapsed_ms(ev0, ev1, C.byref(ms))
    loss = net.loss()
    gflop = net.conv_gflop()
    net.close()
    return dict(wall_s=t1 - t0, gpu_ms=ms.value, loss=loss, first_loss=first_loss,
                gflop_step=gflop, batch=B)


def fed_phase(aetcnn, configs, name, steps, warmup, threads):
    """The same training step fed by the input pipeline (an_feeder, synthetic
    source, `threads` host workers): a fresh batch per step, its host-to-device
    copy overlapped with the previous step.  PCIe-inclusive; not `value`."""
    lib = aetcnn.net_lib()
    lib.an_rand_seed(1)
    B, h, w, c = configs.dims(name)
    net = aetcnn.Network(B, h, w, c)
    configs.build(net, name)
    net.finalize()
    # the reference's augmentation with its [net] defaults (random 1-2x zoom
    # crops, flips, the HSV pass) on every image, as Classifier.train feeds
    feeder = aetcnn.Feeder(net, threads=threads, seed=3, augment=aetcnn.Augment.defaults(w))
    ops = aetcnn.ops()
    for _ in range(warmup):
        feeder.next()
        net.train_step()
    ops.ach_device_sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        feeder.next()
        net.train_step()
    aetcnn.check(ops.ach_device_sync(), "sync")
    dt = time.perf_counter() - t0
    loss = net.loss()
    feeder.close()
    net.close()
    return dict(images_per_s=round(B * steps / dt, 1), ms_per_step=round(dt * 1e3 / steps, 4),
                threads=threads, loss=round(loss, 5),
                source="synthetic images with the reference's default augmentation, a fresh "
                       "batch per step through pinned double buffers")


def time_launch(ops, stream, fn, reps):
    e0, e1 = C.c_void_p(), C.c_void_p()
    ops.ach_event_create(C.byref(e0))
    ops.ach_event_create(C.byref(e1))
    fn()  # warm
    ops.ach_event_record(e0, stream)
    for _ in range(reps):
        fn()
    ops.ach_event_record(e1, stream)
    ms = C.c_float()
    aetcnn_check(ops.ach_event_elapsed_ms(e0, e1, C.byref(ms)), "event")
    ops.ach_event_destroy(e0)
    ops.ach_event_destroy(e1)
    return ms.value / reps


def time_launch_cold(ops, stream, fn, reps, flush):
    """Average time of fn() with the caches flushed before every launch: each
    launch is bracketed by its own events, and flush() (an untimed pass over
    a buffer larger than the 256 MB last-level cache) runs in between."""
    e0, e1 = C.c_void_p(), C.c_void_p()
    ops.ach_event_create(C.byref(e0))
    ops.ach_event_create(C.byref(e1))
    fn()  # warm
    tot = 0.0
    for _ in range(reps):
        flush()
        ops.ach_event_record(e0, stream)
        fn()
        ops.ach_event_record(e1, stream)
        aetcnn_check(ops.ach_stream_sync(stream), "sync")
        ms = C.c_float()
        aetcnn_check(ops.ach_event_elapsed_ms(e0, e1, C.byref(ms)), "event")
        tot += ms.value
    ops.ach_event_destroy(e0)
    ops.ach_event_destroy(e1)
    return tot / reps


def aetcnn_check(rc, what):
    import aetcnn
    aetcnn.check(rc, what)


def config1_inputs(rng, batch, ci, co, hw, k, p):
    """Config 1 operands of one sweep layer: x ~ U[-1,1], w ~ N(0, 0.05),
    dy ~ U[-1,1] (also the inputs of the config-1 parity tests)."""
    oh = (hw + 2 * p - k) + 1
    x = rng.uniform(-1, 1, (batch, ci, hw, hw)).astype(np.float32)
    w = (rng.standard_normal((co, ci, k, k)) * 0.05).astype(np.float32)
    dy = rng.uniform(-1, 1, (batch, co, oh, oh)).astype(np.float32)
    return x, w, dy


def sweep_phase(aetcnn, batch, reps):
    ops = aetcnn.ops()
    D = aetcnn.DeviceArray
    stream = C.c_void_p()
    aetcnn.check(ops.ach_stream_create(C.byref(stream)), "stream")
    rng = np.random.default_rng(0)
    rows = []
    tot_flop = tot_ms = 0.0
    for (ci, co, hw, k, p) in SWEEP:
        d = aetcnn.ConvDesc(batch, ci, hw, hw, co, k, 1, p)
        oh = (hw + 2 * p - k) + 1
        xh, wh, dyh = config1_inputs(rng, batch, ci, co, hw, k, p)
        x, w, dy = D.from_numpy(xh), D.from_numpy(wh), D.from_numpy(dyh)
        y = D((batch, co, oh, oh))
        dx = D((batch, ci, hw, hw))
        dw = D((co, ci, k, k))
        dw.zero()
        wsz = max(ops.ach_conv_fwd_workspace(C.byref(d)),
                  ops.ach_conv_bwd_data_workspace(C.byref(d)),
                  ops.ach_conv_bwd_filter_workspace(C.byref(d)), 256)
        ws = D(wsz // 4)
        flop = 2.0 * batch * co * oh * oh * ci * k * k

        def fwd():
            aetcnn.check(ops.ach_conv_fwd(C.byref(d), x.ptr, w.ptr, y.ptr, ws.ptr, wsz, stream))

        def dgrad():
            aetcnn.check(ops.ach_conv_bwd_data(C.byref(d), dy.ptr, w.ptr, dx.ptr, ws.ptr, wsz,
                                               stream))

        def wgrad():
            aetcnn.check(ops.ach_conv_bwd_filter(C.byref(d), x.ptr, dy.ptr, dw.ptr, ws.ptr, wsz,
                                                 stream))

        t = [time_launch(ops, stream, f, reps) for f in (fwd, dgrad, wgrad)]
        row = dict(shape=f"{ci}->{co}@{hw}x{hw} k{k}", gflop_pass=flop / 1e9,
                   ms=[round(v, 4) for v in t],
                   tflops=[round(flop / (v * 1e-3) / 1e12, 2) for v in t])
        rows.append(row)
        tot_flop += 3 * flop
        tot_ms += sum(t)
        log(f"sweep {row['shape']}: fwd/dgrad/wgrad {row['tflops']} TFLOP/s")
        for a in (x, w, y, dy, dx, dw, ws):
            a.free()
    ops.ach_stream_destroy(stream)
    return rows, tot_flop / (tot_ms * 1e-3) / 1e12


def roofline_phase(aetcnn, batch, reps):
    """The dominant kernel of the training step -- the implicit-GEMM conv
    forward (also used for the stride-1 input gradient) -- on one config-3 /
    config-1 layer, launched `reps` times back to back on its own stream with
    HIP events around the run.  Each ach_conv_fwd call is the filter
    transpose (k_weights_kmajor, ~1% of the time), the GEMM (256 x 128
    tiles, K split in two halves because the 256-tile grid is small) and the
    fixed-order split-K reduction into NCHW (~6%); the average here is the
    whole call, so it under-states the GEMM's own rate."""
    ops = aetcnn.ops()
    D = aetcnn.DeviceArray
    ci, co, hw, k, p = ROOFLINE_SHAPE
    stream = C.c_void_p()
    aetcnn.check(ops.ach_stream_create(C.byref(stream)), "stream")
    d = aetcnn.ConvDesc(batch, ci, hw, hw, co, k, 1, p)
    rng = np.random.default_rng(1)
    x = D.from_numpy(rng.uniform(-1, 1, (batch, ci, hw, hw)).astype(np.float32))
    w = D.from_numpy((rng.standard_normal((co, ci, k, k)) * 0.05).astype(np.float32))
    y = D((batch, co, hw, hw))
    wsz = ops.ach_conv_fwd_workspace(C.byref(d))
    ws = D(wsz // 4 + 64)

    def fwd():
        aetcnn.check(ops.ach_conv_fwd(C.byref(d), x.ptr, w.ptr, y.ptr, ws.ptr, wsz, stream))

    ms = time_launch(ops, stream, fwd, reps)
    flop = 2.0 * batch * co * hw * hw * ci * k * k
    for a in (x, w, y, ws):
        a.free()
    ops.ach_stream_destroy(stream)
    return dict(kernel="k_mfma_gemm<FwdProblem<256, BIm2col3F, true, false>> (conv fwd / dgrad implicit GEMM)",
                shape=f"{ci}->{co}@{hw}x{hw} k{k} b{batch}", flop=flop, ms=ms, reps=reps)


BW_SHAPE = (512, 128, 32, 32)  # config 2: x ~ N(0,1), S = 256 MiB per tensor
SGD_PARAMS = 60_000_000        # config 2: SGD over a 60 M-parameter flat buffer
SGD_HYPER = (0.1, 0.9, 5e-4, 512)  # learning rate, momentum, decay, batch
SOFTMAX_SHAPE = (512, 1000)


def config2_inputs(seed=2):
    """The host arrays of config 2 (also the inputs of its parity tests):
    x and the BN / leaky gradient ~ N(0,1) over [512][128][32][32], the
    2x2 max-pool output gradient, SGD weights / momenta over 60 M
    parameters, 512 x 1000 logits with one-hot labels."""
    B, Cc, H, W = BW_SHAPE
    n = B * Cc * H * W
    rng = np.random.default_rng(seed)
    out = dict(x=rng.standard_normal(n, dtype=np.float32),
               delta=rng.standard_normal(n, dtype=np.float32))
    out["pool_delta"] = rng.standard_normal(n // 4, dtype=np.float32)
    out["sgd_w"] = rng.standard_normal(SGD_PARAMS, dtype=np.float32) * np.float32(0.05)
    out["sgd_v"] = rng.standard_normal(SGD_PARAMS, dtype=np.float32) * np.float32(0.01)
    SB, SK = SOFTMAX_SHAPE
    out["logits"] = rng.standard_normal(SB * SK, dtype=np.float32)
    truth = np.zeros((SB, SK), np.float32)
    truth[np.arange(SB), rng.integers(0, SK, SB)] = 1
    out["truth"] = truth
    return out


def bandwidth_phase(aetcnn, reps):
    """Config 2: the HBM-bound ops on [512][128][32][32] fp32.  Each op is
    launched `reps` times back to back on its own stream between HIP events;
    algorithmic bytes are the minimum traffic the semantics require (BN
    forward 3S with the pre-BN tensor kept, BN backward 5S with x_norm
    recomputed, leaky 2S / 3S, 2x2 max-pool 1.5S each way, SGD 16 bytes per
    parameter); softmax + cross-entropy on 512 x 1000 is reported in us.
    A 1 GiB buffer is read before every timed launch so that no operand
    starts in the 256 MB last-level (Infinity) cache."""
    ops = aetcnn.ops()
    D = aetcnn.DeviceArray
    B, Cc, H, W = BW_SHAPE
    n = B * Cc * H * W
    S = 4.0 * n
    HW = H * W
    stream = C.c_void_p()
    aetcnn.check(ops.ach_stream_create(C.byref(stream)), "stream")
    host = config2_inputs()
    x = D.from_numpy(host["x"])
    delta = D.from_numpy(host["delta"])
    out = D(n)
    chan = [D.from_numpy(np.full(Cc, v, np.float32)) for v in (1.0, 0.0, 0, 0, 0, 0, 0)]
    scales, biases, mean, var, rmean, rvar, supd = chan
    wsz = ops.ach_bn_workspace(B, Cc, HW)
    ws = D(wsz // 4 + 64)
    OH, OW = H // 2, W // 2
    pout = D(B * Cc * OH * OW)
    pidx = D(B * Cc * OH * OW, np.int32)
    pdelta = D.from_numpy(host["pool_delta"])
    LEAKY, LINEAR = aetcnn.LEAKY, aetcnn.LINEAR
    rows = []
    # cache flush: a read-only reduction over 1 GiB (a write pass would leave
    # dirty lines whose write-back then competes with the timed launch)
    flush_n = 1 << 28
    flush_buf = D(flush_n)
    flush_buf.zero()
    flush_out = D(1024)
    fws = ops.ach_bias_grad_workspace(256, 1024, 1024)
    flush_ws = D(max(fws, 256) // 4 + 64)

    def flush():
        aetcnn.check(ops.ach_bias_grad(flush_out.ptr, flush_buf.ptr, 256, 1024, 1024,
                                       flush_ws.ptr, max(fws, 256), stream), "flush")

    def run(name, fn, nbytes):
        ms = time_launch_cold(ops, stream, fn, reps, flush)
        gbs = nbytes / (ms * 1e-3) / 1e9
        rows.append(dict(op=name, ms=round(ms, 5), algorithmic_bytes=nbytes,
                         gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4)))

    chk = aetcnn.check
    run("bn_fwd (stats + normalize, pre-BN tensor kept)",
        lambda: chk(ops.ach_bn_train_fwd_from_x(x.ptr, out.ptr, B, Cc, HW, scales.ptr, biases.ptr,
                                                mean.ptr, var.ptr, rmean.ptr, rvar.ptr, LINEAR,
                                                ws.ptr, wsz, stream)), 3 * S)
    run("bn_bwd (x_norm recomputed)",
        lambda: chk(ops.ach_bn_bwd(delta.ptr, B, Cc, HW, x.ptr, None, mean.ptr, var.ptr,
                                   scales.ptr, biases.ptr, supd.ptr, None, None, LINEAR, ws.ptr,
                                   wsz, stream)), 5 * S)
    run("leaky_fwd", lambda: chk(ops.ach_activate(out.ptr, n, LEAKY, stream)), 2 * S)
    run("leaky_bwd", lambda: chk(ops.ach_gradient(x.ptr, n, LEAKY, delta.ptr, stream)), 3 * S)
    run("maxpool2x2_fwd",
        lambda: chk(ops.ach_maxpool_fwd(x.ptr, B, Cc, H, W, 2, 2, 1, pout.ptr, pidx.ptr,
                                        stream)), 1.5 * S)
    run("maxpool2x2_bwd",
        lambda: chk(ops.ach_maxpool_bwd(pdelta.ptr, pidx.ptr, B, Cc, H, W, 2, 2, 1, delta.ptr,
                                        0, stream)), 1.5 * S)
    for a in (x, delta, out, ws, pout, pidx, pdelta, *chan):
        a.free()
    del host["x"], host["delta"], host["pool_delta"]
    P = SGD_PARAMS
    w = D.from_numpy(host.pop("sgd_w"))
    v = D.from_numpy(host.pop("sgd_v"))
    lr, mom, decay, batch = SGD_HYPER
    run("sgd_update (60 M params)",
        lambda: chk(ops.ach_sgd_update(P, w.ptr, v.ptr, -decay * batch, lr / batch, mom, stream)),
        16.0 * P)
    w.free()
    v.free()
    SB, SK = SOFTMAX_SHAPE
    logits = D.from_numpy(host["logits"])
    dtruth = D.from_numpy(host["truth"])
    prob, sdelta, err, cost = D(SB * SK), D(SB * SK), D(SB * SK), D(4)
    sws = ops.ach_softmax_workspace(SB, 1)
    swsb = D(sws // 4 + 64)
    ms = time_launch_cold(ops, stream, lambda: chk(ops.ach_softmax_xent(
        logits.ptr, SB, SK, 1, 1.0, dtruth.ptr, prob.ptr, sdelta.ptr, err.ptr, cost.ptr,
        swsb.ptr, sws, stream)), reps, flush)
    for a in (logits, dtruth, prob, sdelta, err, cost, swsb, flush_buf, flush_out, flush_ws):
        a.free()
    ops.ach_stream_destroy(stream)
    return rows, round(ms * 1e3, 2)


def copy_calibration_phase(aetcnn, nfloats=1 << 26):
    """One ach_scal over a 256 MiB buffer (reads and writes exactly 256 MiB):
    the reference dispatch that scales rocprofv3's FETCH_SIZE / WRITE_SIZE
    counters to bytes."""
    ops = aetcnn.ops()
    buf = aetcnn.DeviceArray(nfloats)
    buf.zero()
    aetcnn.check(ops.ach_scal(nfloats, 1.0, buf.ptr, None), "scal")
    aetcnn.check(ops.ach_device_sync(), "sync")
    buf.free()
    return nfloats * 4


def cpu_phase(configs, name, batch, steps, parallel=True):
    """The oracle (CPU restatement of the reference CPU path) on a bounded
    sample: `steps` training steps of the same network.  parallel=True is the
    "oracle-parallel" mode (row-parallel GEMM over OpenMP threads, results
    bit-identical to serial); parallel=False is "reference-faithful" (the
    GEMM single-threaded as in the reference, Gemm.c:133)."""
    import oracle_lib
    L = oracle_lib.lib()
    L.or_set_gemm_parallel(1 if parallel else 0)
    L.or_rand_seed(1)
    B, h, w, c = configs.dims(name, batch)
    onet = oracle_lib.OracleNet(B, h, w, c)
    configs.build(onet, name)
    onet.finalize()
    x, truth, _ = configs.synthetic_batch(name, 1234, B)
    onet.train(x, truth)  # warm-up step
    t0 = time.perf_counter()
    for _ in range(steps):
        onet.train(x, truth)
    dt = time.perf_counter() - t0
    threads = L.or_max_threads() if parallel else 1
    onet.close()
    how = (f"row-parallel GEMM on {threads} OpenMP threads" if parallel
           else "single-threaded GEMM (reference-faithful)")
    return dict(value=round(B * steps / dt, 3), unit="images/s", cores=int(threads),
                kind="port",
                sample=f"oracle {name} net, batch {B}, {steps} timed steps after 1 warm-up, "
                       f"{how} ({dt:.1f} s)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="darknet", choices=["darknet", "tiny", "alexnet"])
    ap.add_argument("--sweep-reps", type=int, default=5)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--roofline-reps", type=int, default=20)
    ap.add_argument("--no-bandwidth", action="store_true")
    ap.add_argument("--no-fed", action="store_true",
                    help="skip the input-pipeline (PCIe-inclusive) training measurement")
    ap.add_argument("--bandwidth-only", action="store_true",
                    help="run only the config-2 bandwidth ops and print their rows")
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the roofline probe and the copy calibration dispatch "
                         "(for rocprofv3 counter passes)")
    ap.add_argument("--bandwidth-reps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-batch", type=int, default=128)
    ap.add_argument("--cpu-steps", type=int, default=4)
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU data parallelism is design-only", file=sys.stderr)
        sys.exit(2)

    import aetcnn
    from aetcnn import configs
    ops = aetcnn.ops()
    if ops.ach_device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    aetcnn.check(ops.ach_set_device(0), "set_device")

    if args.roofline_only:
        probe = roofline_phase(aetcnn, 128, args.roofline_reps)
        copy_calibration_phase(aetcnn)
        print(json.dumps({"roofline_probe_ms": probe["ms"], "kernel": probe["kernel"],
                          "shape": probe["shape"]}))
        return
    if args.bandwidth_only:
        rows, softmax_us = bandwidth_phase(aetcnn, args.bandwidth_reps)
        print(json.dumps({"bandwidth_ops": rows, "softmax_xent_512x1000_us": softmax_us}))
        return

    log(f"training phase: {args.config} b128, warmup {args.warmup}, steps {args.steps}")
    tr = train_phase(aetcnn, configs, args.config, args.steps, args.warmup, None)
    ms_step = tr["wall_s"] * 1e3 / args.steps
    ips = tr["batch"] * args.steps / tr["wall_s"]
    step_tflops = tr["gflop_step"] / (ms_step * 1e-3) / 1e3
    log(f"{ms_step:.3f} ms/step ({tr['gpu_ms'] / args.steps:.3f} GPU ms), {ips:.1f} img/s, "
        f"conv {step_tflops:.2f} TFLOP/s, loss {tr['first_loss']:.4f} -> {tr['loss']:.4f}")

    fed = None
    if not args.no_fed:
        fed = fed_phase(aetcnn, configs, args.config, args.steps, args.warmup, 8)
        log(f"fed by the input pipeline: {fed['ms_per_step']:.3f} ms/step, "
            f"{fed['images_per_s']:.1f} img/s")

    sweep_rows, sweep_tflops = [], None
    if not args.no_sweep:
        sweep_rows, sweep_tflops = sweep_phase(aetcnn, 128, args.sweep_reps)
        log(f"conv sweep fwd+dgrad+wgrad: {sweep_tflops:.2f} TFLOP/s")
    bw_rows, softmax_us = [], None
    if not args.no_bandwidth:
        bw_rows, softmax_us = bandwidth_phase(aetcnn, args.bandwidth_reps)
        for r in bw_rows:
            log(f"bandwidth {r['op']}: {r['ms']:.4f} ms, {r['gbs']:.0f} GB/s "
                f"({100 * r['frac']:.1f}% of HBM)")
        log(f"softmax+xent 512x1000: {softmax_us} us")
    probe = roofline_phase(aetcnn, 128, args.roofline_reps)
    copy_calibration_phase(aetcnn)
    log(f"roofline probe {probe['shape']}: {probe['ms']:.4f} ms/launch over {probe['reps']}")

    roofline = None
    if probe:
        ach = probe["flop"] / (probe["ms"] * 1e-3) / 1e12
        roofline = dict(bound="mfma", achieved=round(ach, 3), peak=MFMA_FP32_PEAK_TFLOPS,
                        unit="TFLOP/s", frac=round(ach / MFMA_FP32_PEAK_TFLOPS, 4),
                        traffic=ROOFLINE_TRAFFIC_BYTES, kernel=probe["kernel"],
                        shape=probe["shape"],
                        avg_launch_ms=round(probe["ms"], 5), launches=probe["reps"],
                        flop_per_launch=probe["flop"])

    cpu = cpu_serial = None
    if not args.no_cpu:
        log("cpu baseline (oracle) ...")
        try:
            cpu = cpu_phase(configs, args.config, args.cpu_batch, args.cpu_steps)
            log(f"cpu baseline: {cpu['value']} img/s on {cpu['cores']} threads")
            cpu_serial = cpu_phase(configs, args.config, 16, 1, parallel=False)
            log(f"cpu baseline (reference-faithful): {cpu_serial['value']} img/s")
        except Exception as e:  # the oracle is optional on the box
            log(f"cpu baseline skipped: {e}")

    out = {
        "metric": "train images/s, fp32 32x32 13-conv net b=128; conv fwd+bwd TFLOP/s",
        "value": round(ips, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: seeded uniform [0,1) pixels, uniform labels, one resident batch",
        "config": {"workload": f"{args.config} classifier full training step (fwd+bwd+SGD)",
                   "global_batch": tr["batch"], "input": "3x32x32" if args.config != "alexnet"
                   else "3x227x227", "parallelism": "single GPU"},
        "conv_step_tflops": round(step_tflops, 3),
        "conv_sweep_tflops": None if sweep_tflops is None else round(sweep_tflops, 3),
        "conv_sweep": sweep_rows,
        "loss_first_last": [round(tr["first_loss"], 5), round(tr["loss"], 5)],
        "input_pipeline": fed,
        "bandwidth_ops": {"shape": "x[512][128][32][32] fp32 (config 2)", "ops": bw_rows,
                          "softmax_xent_512x1000_us": softmax_us},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_baseline_reference_faithful": cpu_serial,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
