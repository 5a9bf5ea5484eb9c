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
import csv
import ctypes as C
import glob
import json
import os
import shutil
import signal
import statistics
import subprocess
import sys
import tempfile
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
# Kernel probes, each one config-1 / config-3 layer pass launched back to
# back on its own stream: the conv forward implicit GEMM (the kernel with the
# most time per darknet step; the stride-1 input gradient runs it too) and
# the weight-gradient GEMM (the second most).
PROBES = {
    "fwd": dict(shape=(256, 256, 16, 3, 1), op="fwd",
                kernel="k_mfma_gemm<FwdProblem<128, BIm2col3F, true, false>, 2> "
                       "(conv fwd implicit GEMM, two K groups per workgroup; the stride-1 "
                       "dgrad runs the same loop with one)"),
    "wgrad": dict(shape=(128, 128, 32, 3, 1), op="wgrad",
                  kernel="k_mfma_gemm<WgradProblemC<128, 96, 3>> (conv weight-gradient GEMM)"),
}
CALIB_FLOATS = 1 << 26  # the 256 MiB copy-calibration dispatch


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def train_phase(aetcnn, configs, name, steps, warmup, batch, sustain_s=0.0):
    """Warm-up, then exactly `steps` timed steps between two device
    synchronisations (the headline).  With sustain_s > 0 (the separate
    sustained phase) the same network then trains on in blocks of 50 steps
    until sustain_s seconds have passed, reported as the sustained rate
    (clock and thermal behaviour under load)."""
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
    sustained = None
    if sustain_s > 0:
        n = 0
        s0 = time.perf_counter()
        while time.perf_counter() - s0 < sustain_s:
            for _ in range(50):
                net.train_step()
            aetcnn.check(ops.ach_device_sync(), "sync")
            n += 50
        ds = time.perf_counter() - s0
        sustained = dict(seconds=round(ds, 2), steps=n, images_per_s=round(B * n / ds, 1),
                         ms_per_step=round(ds * 1e3 / n, 4))
    net.close()
    return dict(wall_s=t1 - t0, gpu_ms=ms.value, loss=loss, first_loss=first_loss,
                gflop_step=gflop, batch=B, sustained=sustained)


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


# The shader clock idles low and ramps up only under sustained load.  The
# 256->256@16 forward GEMM timed over 20 launches right after set-up, or
# after a pause of 0.1 s, ran at 114 TFLOP/s; the same 20 launches right
# after 1 s of back-to-back launches at 136 TFLOP/s, with rocm-smi showing
# 2395 MHz (the training step itself runs at 2371-2381 MHz).  So every
# kernel measurement first repeats its call for WARM_S seconds and then
# times it with no pause in between.
WARM_S = 0.3


def warm_up(ops, stream, fn, seconds=WARM_S):
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        aetcnn_check(ops.ach_stream_sync(stream), "sync")


def time_launch(ops, stream, fn, reps):
    e0, e1 = C.c_void_p(), C.c_void_p()
    ops.ach_event_create(C.byref(e0))
    ops.ach_event_create(C.byref(e1))
    warm_up(ops, stream, fn)
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
    warm_up(ops, stream, fn)
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


def sweep_phase(aetcnn, batch, reps, shapes=None):
    ops = aetcnn.ops()
    D = aetcnn.DeviceArray
    stream = C.c_void_p()
    aetcnn.check(ops.ach_stream_create(C.byref(stream)), "stream")
    rng = np.random.default_rng(0)
    rows = []
    tot_flop = tot_ms = 0.0
    for (ci, co, hw, k, p) in (SWEEP if shapes is None else [SWEEP[i] for i in shapes]):
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


def probe_setup(aetcnn, which, batch):
    """Operands of a kernel probe; returns (call, stream, free, flop, shape)."""
    ops = aetcnn.ops()
    D = aetcnn.DeviceArray
    ci, co, hw, k, p = PROBES[which]["shape"]
    stream = C.c_void_p()
    aetcnn.check(ops.ach_stream_create(C.byref(stream)), "stream")
    d = aetcnn.ConvDesc(batch, ci, hw, hw, co, k, 1, p)
    rng = np.random.default_rng(1)
    xh, wh, dyh = config1_inputs(rng, batch, ci, co, hw, k, p)
    x, w, dy = D.from_numpy(xh), D.from_numpy(wh), D.from_numpy(dyh)
    y, dw = D(dyh.shape), D(wh.shape)
    wt = D(wh.shape)
    wsz = max(ops.ach_conv_fwd_workspace(C.byref(d)),
              ops.ach_conv_bwd_filter_workspace(C.byref(d)), 256)
    ws = D(wsz // 4 + 64)
    if PROBES[which]["op"] == "fwd":
        # the k-major filter made once, as the network does once per step
        # for all its layers: each call is then the GEMM launch alone
        job = aetcnn.FilterJob(d, w.ptr, wt.ptr, None)
        aetcnn.check(ops.ach_conv_prepare_filters(1, C.byref(job), stream), "prepare")

        def call():
            aetcnn.check(ops.ach_conv_fwd_prepared(C.byref(d), x.ptr, wt.ptr, y.ptr, ws.ptr, wsz,
                                                   stream))
    else:
        def call():
            aetcnn.check(ops.ach_conv_bwd_filter(C.byref(d), x.ptr, dy.ptr, dw.ptr, ws.ptr, wsz,
                                                 stream))

    def free():
        for a in (x, w, dy, y, dw, ws, wt):
            a.free()
        ops.ach_stream_destroy(stream)
    oh = hw + 2 * p - k + 1
    flop = 2.0 * batch * co * oh * oh * ci * k * k
    return call, stream, free, flop, f"{ci}->{co}@{hw}x{hw} k{k} b{batch}"


def roofline_phase(aetcnn, which, batch, reps):
    """A probe launched `reps` times back to back with HIP events around the
    run on the probe's stream.  The forward call is the GEMM launch alone
    (ach_conv_fwd_prepared on a k-major filter made once: 512 workgroups of
    two K groups over 128 x 128 tiles), so the average is that kernel's; the
    weight-gradient call is the GEMM over chunked K and its fixed-order
    split-K reduction (~5%), whose average is the whole call."""
    ops = aetcnn.ops()
    call, stream, free, flop, shape = probe_setup(aetcnn, which, batch)
    ms = time_launch(ops, stream, call, reps)
    free()
    return dict(kernel=PROBES[which]["kernel"], shape=shape, flop=flop, ms=ms, reps=reps)


def traffic_probe_main(aetcnn, which, calls=3):
    """Child of traffic_phase, run under rocprofv3 --pmc: the copy-calibration
    dispatch, then `calls` probe calls."""
    ops = aetcnn.ops()
    call, stream, free, _, _ = probe_setup(aetcnn, which, 128)
    aetcnn.check(ops.ach_device_sync(), "sync")
    copy_calibration_phase(aetcnn)
    for _ in range(calls):
        call()
    aetcnn.check(ops.ach_device_sync(), "sync")
    free()


def _pmc_dispatches(path):
    """{dispatch id: (kernel name, summed counter value)} of a counter CSV."""
    out = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            k = int(r["Dispatch_Id"])
            name, v = out.get(k, (r["Kernel_Name"], 0.0))
            out[k] = (name, v + float(r["Counter_Value"]))
    return out


def _short_kernel(name):
    name = name.replace("void ", "").replace("ach::", "")
    return name.split(">(")[0] + ">" if "k_mfma_gemm" in name else name.split("(")[0]


def traffic_phase(which, calls=3, timeout=120):
    """HBM bytes per probe call, measured in this run: two rocprofv3 --pmc
    passes (FETCH_SIZE, then WRITE_SIZE) over a child process that runs the
    256 MiB copy calibration (ach_scal: reads and writes exactly 256 MiB) and
    `calls` probe calls; each counter is scaled by what it reads for the
    calibration.  Returns a dict, or None and the reason."""
    prof = shutil.which("rocprofv3")
    if not prof:
        return None, "rocprofv3 not on PATH"
    res, scale, kernels = {}, {}, {}
    tmp = tempfile.mkdtemp(prefix="bench_pmc_")
    try:
        for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
            d = os.path.join(tmp, ctr)
            cmd = [prof, "--pmc", ctr, "-d", d, "-o", "pmc", "--output-format", "csv", "--",
                   sys.executable, os.path.abspath(__file__), "--traffic-probe", which]
            pr = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE,
                                  start_new_session=True, cwd=tmp)
            try:
                _, err = pr.communicate(timeout=timeout)
            except subprocess.TimeoutExpired:
                os.killpg(pr.pid, signal.SIGKILL)
                pr.wait()
                return None, f"rocprofv3 --pmc {ctr} timed out after {timeout} s"
            files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
            if not files:
                tail = err.decode(errors="replace").strip().splitlines()[-1:] if err else []
                return None, f"rocprofv3 --pmc {ctr} wrote no counters (rc {pr.returncode}: " \
                             f"{' '.join(tail)})"
            disp = _pmc_dispatches(files[0])
            ids = sorted(disp)
            cal = [i for i in ids if "k_scal" in disp[i][0]]
            if len(cal) != 1:
                return None, f"{ctr}: expected one calibration dispatch, found {len(cal)}"
            expect_kib = CALIB_FLOATS * 4 / 1024.0
            scale[ctr] = expect_kib / disp[cal[0]][1]
            after = [i for i in ids if i > cal[0]]
            ngemm = sum(1 for i in after if "k_mfma_gemm" in disp[i][0])
            if ngemm != calls:
                return None, f"{ctr}: expected {calls} GEMM dispatches, found {ngemm}"
            tot = 0.0
            for i in after:
                b = disp[i][1] * scale[ctr] * 1024.0 / calls
                tot += b
                kn = _short_kernel(disp[i][0])
                kernels.setdefault(kn, {}).setdefault(ctr, 0.0)
                kernels[kn][ctr] += b
            res[ctr] = tot
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return dict(read_bytes=round(res["FETCH_SIZE"]), write_bytes=round(res["WRITE_SIZE"]),
                bytes=round(res["FETCH_SIZE"] + res["WRITE_SIZE"]),
                scale={k: round(v, 4) for k, v in scale.items()},
                per_kernel={k: {"read": round(v.get("FETCH_SIZE", 0.0)),
                                "write": round(v.get("WRITE_SIZE", 0.0))}
                            for k, v in kernels.items()}), None


def algorithmic_bytes(which, batch=128):
    """Operands each probe call must move at least once: conv forward reads
    x and W and writes y; the weight gradient reads x and dy and writes dW."""
    ci, co, hw, k, p = PROBES[which]["shape"]
    oh = hw + 2 * p - k + 1
    x, w, y = batch * ci * hw * hw, co * ci * k * k, batch * co * oh * oh
    return 4.0 * (x + w + y)


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


def copy_calibration_phase(aetcnn, nfloats=CALIB_FLOATS):
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


def host_cpu():
    """The box's host CPU as BASELINE's protocol asks it stated."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(model=model, nproc=len(os.sched_getaffinity(0)), cpu_count=os.cpu_count(),
                omp_num_threads=os.environ.get("OMP_NUM_THREADS"))


def oracle_native_build():
    """Compiles the oracle with the reference's own flags (-march=native,
    src/makefile:50) on this host into a temporary directory.  Returns
    (library path, None), or (None, reason) to fall back to the prebuilt
    x86-64-v3 library."""
    if not shutil.which("make") or not shutil.which(os.environ.get("CC", "gcc")):
        return None, "no compiler on this host"
    out = tempfile.mkdtemp(prefix="oracle_native_")
    try:
        r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "native",
                            f"OUT={out}"], capture_output=True, text=True, timeout=300)
    except subprocess.TimeoutExpired:
        return None, "native build timed out"
    so = os.path.join(out, "liboracle.so")
    if r.returncode != 0 or not os.path.exists(so):
        return None, f"native build failed: {(r.stderr or r.stdout).strip()[-200:]}"
    return so, None


def cpu_phase(L, configs, name, batch, steps, parallel, build):
    """The oracle (CPU restatement of the reference CPU path) on a bounded
    sample, per BASELINE's protocol: 1 warm-up step, then `steps` steps
    timed one by one on the wall clock, median extrapolated to images/s.
    parallel=True is "oracle-parallel" (row-parallel GEMM over OpenMP
    threads, results bit-identical to serial); parallel=False is
    "reference-faithful" (the GEMM single-threaded as in the reference,
    Gemm.c:133; the elementwise loops still use every OpenMP thread, as the
    reference's own pragmas do)."""
    import oracle_lib
    L.or_set_gemm_parallel(1 if parallel else 0)
    L.or_rand_seed(1)
    B, h, w, c = configs.dims(name, batch)
    onet = oracle_lib.OracleNet(B, h, w, c)
    configs.build(onet, name)
    onet.finalize()
    x, truth, _ = configs.synthetic_batch(name, 1234, B)
    onet.train(x, truth)  # warm-up step
    times = []
    for _ in range(steps):
        t0 = time.perf_counter()
        onet.train(x, truth)
        times.append(time.perf_counter() - t0)
    threads = int(L.or_max_threads())
    onet.close()
    med = statistics.median(times)
    how = (f"GEMM row-parallel on {threads} OpenMP threads" if parallel
           else f"GEMM single-threaded (reference-faithful), elementwise loops on {threads} "
                f"OpenMP threads")
    return dict(value=round(B / med, 3), unit="images/s", cores=threads,
                gemm_threads=threads if parallel else 1, kind="port", build=build,
                step_s=[round(v, 3) for v in times],
                sample=f"oracle {name} net, batch {B}: 1 warm-up step, then the median of "
                       f"{steps} timed steps ({med:.2f} s/step); {how}; built {build}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="darknet", choices=["darknet", "tiny", "alexnet"])
    ap.add_argument("--sweep-reps", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--sweep-only", action="store_true",
                    help="run only the config-1 sweep and print its rows (for rocprofv3)")
    ap.add_argument("--sweep-shapes", default=None,
                    help="comma-separated indices into the config-1 sweep (default: all)")
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
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the full-step timing of the two configs besides --config")
    ap.add_argument("--cpu-batch", type=int, default=128)
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--cpu-faithful-batch", type=int, default=16)
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 --pmc passes that measure roofline.traffic")
    ap.add_argument("--traffic-probe", choices=sorted(PROBES),
                    help="(internal) run one probe's traffic child under rocprofv3")
    ap.add_argument("--sustain-s", type=float, default=10.0,
                    help="seconds of further training after the timed steps, reported as the "
                         "sustained rate (0 to skip)")
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

    if args.traffic_probe:
        traffic_probe_main(aetcnn, args.traffic_probe)
        return
    if args.roofline_only:
        rows = {}
        for which in PROBES:
            probe = roofline_phase(aetcnn, which, 128, args.roofline_reps)
            rows[which] = {"ms": probe["ms"], "kernel": probe["kernel"], "shape": probe["shape"]}
        copy_calibration_phase(aetcnn)
        print(json.dumps({"roofline_probes": rows}))
        return
    if args.sweep_only:
        shapes = None if args.sweep_shapes is None else [int(s) for s in args.sweep_shapes.split(",")]
        rows, tf = sweep_phase(aetcnn, 128, args.sweep_reps, shapes)
        print(json.dumps({"conv_sweep": rows, "conv_sweep_tflops": round(tf, 3)}))
        return
    if args.bandwidth_only:
        rows, softmax_us = bandwidth_phase(aetcnn, args.bandwidth_reps)
        copy_calibration_phase(aetcnn)  # scales rocprofv3 counter passes over this run
        print(json.dumps({"bandwidth_ops": rows, "softmax_xent_512x1000_us": softmax_us}))
        return

    log(f"training phase: {args.config} b128, warmup {args.warmup}, steps {args.steps}")
    tr = train_phase(aetcnn, configs, args.config, args.steps, args.warmup, None)
    ms_step = tr["wall_s"] * 1e3 / args.steps
    ips = tr["batch"] * args.steps / tr["wall_s"]
    step_tflops = tr["gflop_step"] / (ms_step * 1e-3) / 1e3
    log(f"{ms_step:.3f} ms/step ({tr['gpu_ms'] / args.steps:.3f} GPU ms), {ips:.1f} img/s, "
        f"conv {step_tflops:.2f} TFLOP/s, loss {tr['first_loss']:.4f} -> {tr['loss']:.4f}")
    # the other two full-step configs (BASELINE configs 0 / 3 / 4), each timed
    # the same way at batch 128: the headline stays --config's
    other_steps = {}
    if not args.no_other_configs:
        for name in ("tiny", "darknet", "alexnet"):
            if name == args.config:
                continue
            o = train_phase(aetcnn, configs, name, args.steps, args.warmup, None)
            oms = o["wall_s"] * 1e3 / args.steps
            otf = o["gflop_step"] / (oms * 1e-3) / 1e3
            other_steps[f"{name}_step"] = dict(
                ms_per_step=round(oms, 4), images_per_s=round(o["batch"] * args.steps / o["wall_s"], 1),
                gpu_ms_per_step=round(o["gpu_ms"] / args.steps, 4), batch=o["batch"],
                steps=args.steps, warmup=args.warmup, conv_gflop_per_step=round(o["gflop_step"], 2),
                conv_tflops=round(otf, 3), frac_of_fp32_mfma_peak=round(otf / MFMA_FP32_PEAK_TFLOPS, 4),
                loss_first_last=[round(o["first_loss"], 5), round(o["loss"], 5)])
            log(f"{name} b{o['batch']}: {oms:.3f} ms/step, "
                f"{other_steps[name + '_step']['images_per_s']} img/s, conv {otf:.2f} TFLOP/s")
    # kernel measurements next, before the long fed and sustained runs heat the
    # GPU and lower its clocks
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
    rooflines = {}
    for which in PROBES:
        probe = roofline_phase(aetcnn, which, 128, args.roofline_reps)
        log(f"roofline probe {which} {probe['shape']}: {probe['ms']:.4f} ms/launch over "
            f"{probe['reps']}")
        ach = probe["flop"] / (probe["ms"] * 1e-3) / 1e12
        traffic, why = (None, "--no-traffic") if args.no_traffic else traffic_phase(which)
        if traffic:
            log(f"traffic {which}: {traffic['read_bytes'] / 1e6:.1f} MB read + "
                f"{traffic['write_bytes'] / 1e6:.1f} MB written per call "
                f"(algorithmic {algorithmic_bytes(which) / 1e6:.1f} MB)")
        else:
            log(f"traffic {which}: not measured ({why})")
        rooflines[which] = dict(
            bound="mfma", achieved=round(ach, 3), peak=MFMA_FP32_PEAK_TFLOPS, unit="TFLOP/s",
            frac=round(ach / MFMA_FP32_PEAK_TFLOPS, 4),
            traffic=traffic["bytes"] if traffic else None,
            kernel=probe["kernel"], shape=probe["shape"], avg_launch_ms=round(probe["ms"], 5),
            launches=probe["reps"], flop_per_launch=probe["flop"],
            algorithmic_bytes=algorithmic_bytes(which),
            traffic_detail=traffic if traffic else {"unmeasured": why})

    fed = None
    if not args.no_fed:
        fed = fed_phase(aetcnn, configs, args.config, args.steps, args.warmup, 8)
        log(f"fed by the input pipeline: {fed['ms_per_step']:.3f} ms/step, "
            f"{fed['images_per_s']:.1f} img/s")
    sustained = None
    if args.sustain_s > 0:
        sustained = train_phase(aetcnn, configs, args.config, args.steps, args.warmup, None,
                                args.sustain_s)["sustained"]
        log(f"sustained over {sustained['seconds']} s: {sustained['images_per_s']} img/s")

    cpu = cpu_serial = None
    host = host_cpu()
    if not args.no_cpu:
        log(f"cpu baseline (oracle) on {host['model']}, nproc {host['nproc']} ...")
        so = None
        try:
            import oracle_lib
            so, why = oracle_native_build()
            build = "-O3 -ffast-math -march=native -fopenmp (the reference's flags)"
            if so:
                oracle_lib.set_library(so)
            else:
                build = f"-O3 -ffast-math -march=x86-64-v3 -fopenmp (prebuilt; {why})"
            L = oracle_lib.lib()
            cpu = cpu_phase(L, configs, args.config, args.cpu_batch, args.cpu_steps, True, build)
            log(f"cpu baseline: {cpu['value']} img/s on {cpu['cores']} threads")
            cpu_serial = cpu_phase(L, configs, args.config, args.cpu_faithful_batch,
                                   args.cpu_steps, False, build)
            log(f"cpu baseline (reference-faithful): {cpu_serial['value']} img/s")
        except Exception as e:  # the oracle is optional on the box
            log(f"cpu baseline skipped: {e}")
        if so:  # loaded already; the scratch build directory can go
            shutil.rmtree(os.path.dirname(so), ignore_errors=True)
        for c in (cpu, cpu_serial):
            if c:
                c["host"] = host

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
        "sustained": sustained,
        **other_steps,
        "roofline": rooflines["fwd"],
        "roofline_wgrad": rooflines["wgrad"],
        "cpu_baseline": cpu,
        "cpu_baseline_reference_faithful": cpu_serial,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
