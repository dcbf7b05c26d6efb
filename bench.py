"""Benchmark: AlexNet-224 fp32 batch-128 training step on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]

One step = forward (5 conv + 3 maxpool + 3 linear), softmax-CE, the full
backward (conv dW/db/dX implicit-GEMM MFMA kernels, maxpool routing, linear
GEMMs, bias/ReLU gradients) and an AdamW update (lr 1e-4, wd 0.01, element
clip 1.0) of all 61.1 M parameters, through the drop-in ``nn_engine`` API.
Inputs are synthetic and already resident in device memory when the timed
region starts.  Prints ONE JSON line on stdout; diagnostics go to stderr.

Roofline object: the conv backward of every layer of one step -- each
ConvBackwardFused call as a whole: the masked NHWC transpose of dy with its
bias-gradient partials, the bias-gradient sum, the filter re-layout, the dW and
dX implicit-GEMM kernels and their split-K finishes -- timed with HIP events on
the engine stream over the timed region; achieved = algorithmic FLOPs
(2*OC*C*k*k*B*OH*OW per dW and per dX; c1 has no dX since the input needs no
gradient) / summed call time.  The GEMM kernels alone are reported beside it.

A second timed pass uploads a fresh batch from host memory every step, as the
reference's training loop does (train_alexnet.py:110); its rate is reported as
`value_upload_inclusive`, never as `value`.

cpu_baseline: the float64 NumPy oracle running the same train step on a
256-image sample on the host, timed on this machine.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

MFMA_FP32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix peak
HBM_PEAK_GBS = 8000.0

CONVS = [  # name, inC, outC, k, stride, pad, input H/W
    ("c1", 3, 64, 11, 4, 2, 224),
    ("c2", 64, 192, 5, 1, 2, 27),
    ("c3", 192, 384, 3, 1, 1, 13),
    ("c4", 384, 256, 3, 1, 1, 13),
    ("c5", 256, 256, 3, 1, 1, 13),
]
FCS = [("l1", 9216, 4096, True), ("l2", 4096, 4096, True), ("l3", 4096, 1000, False)]
BATCH = 128
SEED = 5 * 1000
# The roofline family, the only one timed (HIP events) during the timed
# steps: every event pair on the stream costs a few microseconds of idle GPU,
# so the per-family breakdown comes from a separate pass after the timed one.
ROOFLINE_FAMILY = "conv_bwd"
BREAKDOWN_FAMILIES = ("conv_dw", "conv_dx", "conv_fwd", "gemm", "maxpool_fwd", "maxpool_bwd", "adam")


TRAFFIC_PROFILE = os.path.join(REPO, "profiles", "alexnet224_b128_conv_bwd_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per ConvBackwardFused call (every kernel of the call) from
    the committed rocprofv3 FETCH_SIZE / WRITE_SIZE measurement, and the
    algorithmic bytes per call; (None, None) when the summary is absent."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None, None
    vals = {}
    for key in ("conv_bwd_hbm_bytes_per_step", "conv_bwd_calls_per_step",
                "conv_bwd_algorithmic_bytes_per_step"):
        m = re.search(key + r": (\d+)", text)
        if not m:
            return None, None
        vals[key] = int(m.group(1))
    n = vals["conv_bwd_calls_per_step"]
    return vals["conv_bwd_hbm_bytes_per_step"] / n, vals["conv_bwd_algorithmic_bytes_per_step"] / n


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def conv_bwd_flops(batch):
    """Algorithmic conv-backward FLOPs of one step: dW for every layer, dX for
    every layer except c1 (the network input needs no gradient)."""
    tot = 0.0
    for name, cin, cout, k, s, p, hw in CONVS:
        o = (hw + 2 * p - k) // s + 1
        f = 2.0 * cout * cin * k * k * batch * o * o
        tot += f * (1 if name == "c1" else 2)
    return tot


def he_params(rng):
    p = {}
    for name, cin, cout, k, _, _, _ in CONVS:
        p[name + ".w"] = (rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
        p[name + ".b"] = np.zeros(cout, np.float32)
    for name, fin, fout, _ in FCS:
        p[name + ".w"] = (rng.standard_normal((fin, fout)) * np.sqrt(2.0 / fin)).astype(np.float32)
        p[name + ".b"] = np.zeros(fout, np.float32)
    return p


def build_alexnet(nn, params):
    class AlexNet(nn.Model):
        def __init__(self):
            super().__init__()
            for name, cin, cout, k, s, p, _ in CONVS:
                layer = nn.ConvLayer.__new__(nn.ConvLayer)
                layer.filters = nn.Tensor(params[name + ".w"].copy(), requires_grad=True, track=False)
                layer.bias = nn.Tensor(params[name + ".b"].copy(), requires_grad=True, track=False)
                layer.stride, layer.padding = s, p
                setattr(self, name, layer)
            for name, fin, fout, _ in FCS:
                layer = nn.Linear.__new__(nn.Linear)
                layer.w = nn.Tensor(params[name + ".w"].copy(), requires_grad=True, track=False)
                layer.b = nn.Tensor(params[name + ".b"].copy(), requires_grad=True, track=False)
                setattr(self, name, layer)

        def forward(self, xb):
            x = self.c1(xb, relu=True)
            x = nn.maxpool2d(x, pool_size=3, stride=2)
            x = self.c2(x, relu=True)
            x = nn.maxpool2d(x, pool_size=3, stride=2)
            x = self.c3(x, relu=True)
            x = self.c4(x, relu=True)
            x = self.c5(x, relu=True)
            x = nn.maxpool2d(x, pool_size=3, stride=2)
            x = nn.flatten(x)
            x = self.l1(x, relu=True)
            x = self.l2(x, relu=True)
            return self.l3(x)

    return AlexNet()


def _blas_info():
    """(threads the host BLAS uses, its name and version)."""
    threads = os.cpu_count() or 1
    blas = "unknown"
    try:
        from threadpoolctl import threadpool_info
        info = [i for i in threadpool_info() if i.get("user_api") == "blas"]
        if info:
            threads = int(info[0].get("num_threads", threads))
            blas = f"{info[0].get('internal_api')} {info[0].get('version')}"
    except Exception:
        pass
    return threads, blas


def _time_oracle(fn, images_per_call, budget_s=10.0):
    """Call fn() until budget_s seconds have passed (at least once); returns
    (images per second, calls, seconds)."""
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            return images_per_call * calls / dt, calls, dt


def cpu_baseline_config(cid, budget_s=10.0):
    """The float64 oracle on a bounded sample of configuration `cid`'s step,
    timed on the host (about budget_s seconds); same seeds as the GPU run."""
    from oracle import models as OM
    threads, blas = _blas_info()
    r = np.random.default_rng
    if cid == 1:
        P = OM.he_params(r(1001), OM.LENET_CONVS, OM.LENET_FCS)
        x = r(1000).standard_normal((64, 1, 28, 28)).astype(np.float32)
        y = r(1002).integers(0, 10, 64).astype(np.float32)
        n, what = 64, "LeNet-5 train steps (fwd + bwd + SGD) at batch 64"
        fn = lambda: OM.lenet_step(P, x, y)
    elif cid == 2:
        n = 8
        w = (r(2001).standard_normal((128, 64, 3, 3)) * np.sqrt(2.0 / 576)).astype(np.float32)
        x = r(2000).standard_normal((n, 64, 56, 56)).astype(np.float32)
        dy = r(2002).standard_normal((n, 128, 56, 56)).astype(np.float32)
        what = f"conv backward (mask, dW, db, dX) of {n} of the 128 images"
        fn = lambda: OM.conv_backward_step(x, w, dy)
    elif cid == 3:
        n = 2
        P = OM.mobilenet_stack_params(r(3001))
        x = r(3000).standard_normal((n, 16, 112, 112)).astype(np.float32)
        y = r(3002).integers(0, 10, n).astype(np.float32)
        what = f"MobileNetV2-stack train steps (fwd + bwd + SGD) on {n} of the 64 images"
        fn = lambda: OM.mobilenet_stack_step(P, x, y)
    else:
        n = 1
        P = OM.unet_params(r(4001))
        x = r(4000).random((n, 3, 256, 256)).astype(np.float32)
        m = (r(4002).random((n, 1, 32, 32)) < 0.3).astype(np.float32)
        t = m.repeat(8, axis=2).repeat(8, axis=3)
        what = f"UNet-base16 train steps (fwd + Dice + bwd + clip + Adam) on {n} of the 8 images"
        fn = lambda: OM.unet_step(P, x, t)
    rate, calls, dt = _time_oracle(fn, n, budget_s)
    return {"value": round(rate, 3), "unit": "img/s", "cores": threads, "kind": "port",
            "sample": f"{calls} x {what}, float64 NumPy oracle, {blas}, {dt:.1f} s"}


def cpu_baseline(sample=256):
    """Time the float64 oracle on the same train step for `sample` images."""
    from oracle import models as OM
    threads, blas = _blas_info()
    rng = np.random.default_rng(SEED + 1)
    params = he_params(rng)
    x = np.random.default_rng(SEED).standard_normal((sample, 3, 224, 224)).astype(np.float32)
    y = np.random.default_rng(SEED + 2).integers(0, 1000, sample).astype(np.float32)
    t0 = time.perf_counter()
    OM.alexnet_step(params, x, y, t=1, lr=1e-4, wd=0.01, clip=1.0)
    dt = time.perf_counter() - t0
    return {"value": sample / dt, "unit": "img/s", "cores": threads, "kind": "port",
            "sample": f"one AlexNet-224 train step (fwd+bwd+AdamW) on {sample} images, "
                      f"float64 NumPy oracle, {blas}, {dt:.1f} s"}


HBM_PEAK_BYTES_PER_S = HBM_PEAK_GBS * 1e9


def memory_suite(reps=10, trials=5):
    """Backward memory-bound kernels at the shapes of the benchmark networks,
    each driven through the same dispatch the API's backward makes.  One JSON
    line per kernel: algorithmic bytes per launch (each required tensor read
    or written once), the time per launch of `reps` back-to-back launches
    (one HIP-event pair around them; the median of `trials` such runs), GB/s
    and fraction of 8 TB/s; and the same for a single launch with cold caches
    (`us_cold`, `frac_hbm_cold`): before each timed launch a 1 GiB read pass
    (the norm's sum of squares over a 1 GiB tensor) evicts the operands from
    the 256 MiB MALL and the L2s, so the launch reads HBM, as a kernel inside
    a training step whose working set exceeds the MALL does."""
    from directcompute_torch_amd import nn_engine as nn
    lib = nn.lib
    rng = np.random.default_rng(SEED + 7)
    f2u = nn.float_to_uint
    held = []

    def buf(shape, kind="normal"):
        n = int(np.prod(shape))
        if kind == "normal":
            a = rng.standard_normal(n).astype(np.float32)
        elif kind == "unit":
            a = rng.random(n).astype(np.float32)
        else:
            a = np.zeros(n, np.float32)
        h = lib.CreateBuffer(a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n)
        held.append(h)
        return h

    def prof(fam):
        n, ms, fl, by = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        if not lib.GetProfile(fam.encode(), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl), ctypes.byref(by)):
            return 0, 0.0
        return n.value, ms.value

    out = []
    flush_n = 1 << 28                           # 1 GiB of floats, read by the cold-cache flush
    flush_h = lib.CreateBuffer(None, flush_n)
    held.append(flush_h)
    lib.ClearBuffer(flush_h)
    flush_g = (ctypes.c_void_p * 1)(flush_h)
    flush_s = (ctypes.c_uint * 1)(flush_n)

    def flush():
        lib.ClipGradNorm(flush_g, flush_s, 1, 1e30)   # reads 1 GiB; a zero norm scales nothing

    def run(kernel, family, shape, nbytes, fn, per_launch=False):
        # One event pair around `reps` back-to-back launches (an event pair per
        # launch would add its own few microseconds of idle GPU to each), or,
        # with per_launch, the family's own event pair inside each call (for
        # calls that launch more than the kernel measured).  The median of
        # `trials` such measurements is reported (single runs vary by a few
        # percent from run to run).
        fn()
        lib.SyncGPU()
        per = []
        for _ in range(trials):
            lib.ResetProfile()
            if per_launch:
                lib.SetProfiling(1)
            else:
                lib.BeginProfileRegion(family.encode(), 0.0, float(nbytes) * reps)
            for _ in range(reps):
                fn()
            if per_launch:
                lib.SyncGPU()
                lib.SetProfiling(0)
            else:
                lib.EndProfileRegion()
            lib.SyncGPU()
            n, ms = prof(family)
            per.append(ms / (max(n, 1) if per_launch else reps) * 1e3)
        us = float(np.median(per))
        gbps = nbytes / (us * 1e-6) / 1e9 if us > 0 else 0.0
        cold = []
        for _ in range(trials):
            flush()
            lib.SyncGPU()
            lib.ResetProfile()
            if per_launch:
                lib.SetProfiling(1)
            else:
                lib.BeginProfileRegion(family.encode(), 0.0, float(nbytes))
            fn()
            if per_launch:
                lib.SyncGPU()
                lib.SetProfiling(0)
            else:
                lib.EndProfileRegion()
            lib.SyncGPU()
            n, ms = prof(family)
            cold.append(ms / max(n, 1) * 1e3 if per_launch else ms * 1e3)
        us_c = float(np.median(cold))
        gbps_c = nbytes / (us_c * 1e-6) / 1e9 if us_c > 0 else 0.0
        rec = {"suite": "memory", "kernel": kernel, "family": family, "shape": list(shape),
               "bytes_per_launch": int(nbytes), "us": round(us, 2), "GB/s": round(gbps, 1),
               "frac_hbm": round(gbps * 1e9 / HBM_PEAK_BYTES_PER_S, 4),
               "us_cold": round(us_c, 2), "GB/s_cold": round(gbps_c, 1),
               "frac_hbm_cold": round(gbps_c * 1e9 / HBM_PEAK_BYTES_PER_S, 4)}
        out.append(rec)
        print(json.dumps(rec), flush=True)

    def ew(name, shape, unary_saved="normal", extra=None):
        n = int(np.prod(shape))
        g, x, o = buf(shape), buf(shape, unary_saved), buf(shape, "zero")
        cb = dict(u1=n)
        if extra:
            cb.update(extra)
        run(name, name, shape, 12 * n,
            lambda: nn._dispatch(name.encode(), (g, x), (o,), (n + 255) // 256, 1, 1, **cb))

    mb = (64, 96, 112, 112)      # MobileNetV2 IR stack b64: 96-channel expand at 112^2
    ew("relu6_grad", mb)
    ew("relu_grad", mb)
    ew("leaky_relu_grad", mb, extra=dict(u2=f2u(0.1)))
    ew("sigmoid_grad", (8, 1, 256, 256), "unit")

    un = (8, 16, 256, 256)       # UNet-base16 b8 level-1 activation
    n = int(np.prod(un))
    acc, g = buf(un), buf(un)
    run("grad_accum", "grad_accum", un, 12 * n,
        lambda: nn._dispatch(b"grad_accum", (g,), (acc,), (n + 255) // 256, 1, 1, u1=n))

    # BatchNorm backward (reduce + dx)
    B, C, H, W = mb
    S = H * W
    n = B * C * S
    x, dy = buf(mb), buf(mb)
    mean, var, gamma = buf((C,), "zero"), buf((C,), "unit"), buf((C,), "unit")
    dg, db, dx = buf((C,), "zero"), buf((C,), "zero"), buf(mb, "zero")
    rmean, rvar = buf((C,), "zero"), buf((C,), "unit")   # running statistics
    nn._dispatch(b"batchnorm_mean_var", (x,), (mean, var, rmean, rvar),
                 C, 1, 1, u1=B, u2=C, u3=S, u4=1, u5=f2u(0.1), cbSize=20)
    cb = dict(u1=B, u2=C, u3=S, u4=f2u(1e-5))
    run("batchnorm_backward_reduce", "bn_bwd_reduce", mb, 8 * n,
        lambda: nn._dispatch(b"batchnorm_backward_reduce", (x, dy, mean, var), (dg, db), C, 1, 1, **cb))
    run("batchnorm_backward_dx", "bn_bwd_dx", mb, 12 * n,
        lambda: nn._dispatch(b"batchnorm_backward_dx", (x, dy, mean, var, gamma, dg, db), (dx,),
                             (n + 255) // 256, 1, 1, **cb))
    # The running statistics are made once: a buffer created inside the timed
    # launches would time its allocation and host upload too.
    run("batchnorm_mean_var", "bn_stats", mb, 4 * n,
        lambda: nn._dispatch(b"batchnorm_mean_var", (x,), (mean, var, rmean, rvar),
                             C, 1, 1, u1=B, u2=C, u3=S, u4=1, u5=f2u(0.1), cbSize=20))

    # Depthwise 3x3 backward: stride 1 (hidden 144 at 56^2) and stride 2 (96 at 112^2 -> 56^2)
    for (B, C, H, W, s) in ((64, 144, 56, 56, 1), (64, 96, 112, 112, 2)):
        OH = (H + 2 - 3) // s + 1
        nx, ny = B * C * H * W, B * C * OH * OH
        xs, dys, fs = buf((B, C, H, W)), buf((B, C, OH, OH)), buf((C, 1, 3, 3))
        dxs, dfs, dbs = buf((B, C, H, W), "zero"), buf((C, 1, 3, 3), "zero"), buf((C,), "zero")
        cb = dict(u1=B, u2=C, u3=H, u4=W, u5=3, u6=3, u7=s, u8=1, u9=OH, cbSize=36)
        run(f"depthwise_conv_backward_input_s{s}", "dw_bwd_input", (B, C, H, W), 4 * (nx + ny),
            lambda: nn._dispatch(b"depthwise_conv_backward_input", (dys, fs), (dxs,), (nx + 255) // 256, 1, 1, **cb))
        run(f"depthwise_conv_backward_filter_s{s}", "dw_bwd_filter", (B, C, H, W), 4 * (nx + ny),
            lambda: nn._dispatch(b"depthwise_conv_backward_filter", (dys, xs), (dfs, dbs), C, 1, 1, **cb))

    # Max-pool backward: UNet 2x2 s2 and AlexNet c1 3x3 s2.  The indices of one
    # fused forward serve every launch: each backward consumes one reference,
    # so the handle carries one per launch.
    for (shape, k, st) in (((8, 16, 256, 256), 2, 2), ((128, 64, 55, 55), 3, 2)):
        B, C, H, W = shape
        OH, OW = (H - k) // st + 1, (W - k) // st + 1
        xin, dz = buf(shape), buf((B, C, OH, OW))
        nx, no = B * C * H * W, B * C * OH * OW
        pidx = ctypes.c_void_p()
        held.append(lib.MaxPoolForwardFused(xin, B, C, H, W, k, st, ctypes.byref(pidx)))
        for _ in range(trials * (reps + 1) + 1):   # warm runs, cold runs and the first call
            lib.AddRefBuffer(pidx.value)

        def mp(idx=pidx.value, dz=dz, B=B, C=C, OH=OH, OW=OW, nx=nx):
            lib.ReleaseBuffer(lib.MaxPoolBackwardFused(dz, idx, B, C, OH, OW, nx))
        run(f"maxpool_backward_{k}x{k}s{st}", "maxpool_bwd", shape, 8 * no + 4 * nx, mp)
        lib.ReleaseBuffer(pidx.value)

    # UNet decoder: nearest upsample x2 backward, concat backward (slice)
    B, C, H, W = 8, 32, 128, 128
    dyu, dxu = buf((B, C, 2 * H, 2 * W)), buf((B, C, H, W), "zero")
    run("upsample_backward", "upsample_bwd", (B, C, H, W), 4 * B * C * H * W * 5,
        lambda: nn._dispatch(b"upsample_backward", (dyu,), (dxu,), (B * C * H * W + 255) // 256, 1, 1,
                             u1=B, u2=C, u3=H, u4=W, u5=2 * H, u6=2 * W, u7=2, u8=2, cbSize=32))
    B, Ct, S = 8, 32, 256 * 256
    dyc, sl = buf((B, Ct, 256, 256)), buf((B, 16, 256, 256), "zero")
    run("slice", "slice", (B, 16, 256, 256), 8 * B * 16 * S,
        lambda: nn._dispatch(b"slice", (dyc,), (sl,), (B * 16 * S + 255) // 256, 1, 1,
                             u1=B, u2=16, u3=S, u4=Ct, u5=16, cbSize=20))

    # Global-average-pool backward: broadcast g/S over [64, 96, 112, 112]
    B, C, H, W = mb
    gg, dxg = buf((B, C)), buf(mb, "zero")
    run("global_avg_pool_backward", "gap_bwd", mb, 4 * B * C * H * W,
        lambda: nn._dispatch(b"global_avg_pool_backward", (gg,), (dxg,), (B * C * H * W + 255) // 256, 1, 1,
                             u1=B, u2=C, u3=H * W))

    # Dice loss gradient, UNet output [8, 1, 256, 256]
    B, size = 8, 256 * 256
    pred, tgt, sums, gd = buf((B, size), "unit"), buf((B, size), "unit"), buf((B * 3,), "zero"), buf((B, size), "zero")
    nn._dispatch(b"dice_loss_sums", (pred, tgt), (sums,), B, 1, 1, u1=B, u2=size)
    run("dice_loss_grad", "dice_loss_grad", (B, 1, 256, 256), 12 * B * size,
        lambda: nn._dispatch(b"dice_loss_grad", (pred, tgt, sums), (gd,), (B * size + 255) // 256, 1, 1,
                             u1=B, u2=size))

    # Conv backward G pass (mask + NHWC transpose + bias partials) at AlexNet c1/c2 shapes,
    # through ConvBackwardFused with only db requested.
    for name, cin, cout, k, s, p, hw in CONVS[:2]:
        o = (hw + 2 * p - k) // s + 1
        xc, wc, bc = buf((BATCH, cin, hw, hw)), buf((cout, cin, k, k)), buf((cout,), "zero")
        yc = lib.ConvForwardFused(xc, wc, bc, BATCH, cin, hw, hw, cout, k, k, s, p, 1, None)
        held.append(yc)
        dyc2 = buf((BATCH, cout, o, o))
        cpad = (cout + 3) // 4 * 4

        def gpass(xc=xc, wc=wc, yc=yc, dyc2=dyc2, cin=cin, hw=hw, cout=cout, k=k, s=s, p=p):
            pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
            lib.ConvBackwardFused(dyc2, yc, xc, wc, None, BATCH, cin, hw, hw, cout, k, k, s, p, 1,
                                  0, 0, 1, ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
            lib.ReleaseBuffer(pdb.value)
        run(f"conv_grad_reshape_relu_{name}", "conv_grad_nhwc", (BATCH, cout, o, o),
            4 * BATCH * o * o * (2 * cout + cpad), gpass, per_launch=True)

    # Optimisers over AlexNet's 61.1 M parameters (16 tensors)
    shapes = [(c[2], c[1], c[3], c[3]) for c in CONVS] + [(c[2],) for c in CONVS] + \
             [(f[1], f[2]) for f in FCS] + [(f[2],) for f in FCS]
    ps = [buf(sh, "unit") for sh in shapes]
    gs = [buf(sh) for sh in shapes]
    ms = [buf(sh, "zero") for sh in shapes]
    vs = [buf(sh, "zero") for sh in shapes]
    sizes = [int(np.prod(sh)) for sh in shapes]
    P = len(shapes)
    arr = lambda hs: (ctypes.c_void_p * P)(*hs)
    pa, ga, ma, va = arr(ps), arr(gs), arr(ms), arr(vs)
    sa = (ctypes.c_uint * P)(*sizes)
    tot = sum(sizes)
    run("SGDBatch", "sgd", (tot,), 12 * tot, lambda: lib.SGDBatch(pa, ga, sa, P, 1e-9, 1.0))
    run("AdamBatch", "adam", (tot,), 28 * tot,
        lambda: lib.AdamBatch(pa, ga, ma, va, sa, P, 1e-9, 0.9, 0.999, 1e-8, 0.0, 1.0))
    run("ClipGradNorm: sum of squares", "grad_norm", (tot,), 4 * tot,
        lambda: lib.ClipGradNorm(ga, sa, P, 1e30), per_launch=True)

    for h in held:
        lib.ReleaseBuffer(h)
    fr = [r["frac_hbm"] for r in out if r["bytes_per_launch"] >= 64 << 20]
    fc = [r["frac_hbm_cold"] for r in out if r["bytes_per_launch"] >= 64 << 20]
    print(json.dumps({"suite": "memory", "summary": {
        "kernels": len(out), "kernels_over_64MiB": len(fr),
        "median_frac_hbm_over_64MiB": round(float(np.median(fr)), 4) if fr else None,
        "min_frac_hbm_over_64MiB": round(float(min(fr)), 4) if fr else None,
        "median_frac_hbm_cold_over_64MiB": round(float(np.median(fc)), 4) if fc else None,
        "min_frac_hbm_cold_over_64MiB": round(float(min(fc)), 4) if fc else None}}), flush=True)


def _prof_all(lib):
    """Every kernel family's (launches, ms, flops, bytes) recorded so far."""
    fams = ("conv_bwd", "conv_fwd", "conv_dw", "conv_dx", "gemm", "maxpool_fwd", "maxpool_bwd", "bn_stats",
            "bn_stats_side", "bn_fwd", "bn_bwd_reduce", "bn_bwd_reduce_side", "bn_bwd_dx",
            "dw_bwd_input", "dw_bwd_filter",
            "gap_bwd", "upsample", "upsample_bwd", "dice_loss_grad", "bias_grad", "sgd", "adam",
            "grad_norm",
            "clip_scale", "relu", "relu6", "relu_grad", "relu6_grad", "sigmoid_grad", "grad_accum",
            "slice", "conv_grad_nhwc", "nhwc")
    out = {}
    for f in fams:
        n, ms, fl, by = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        if lib.GetProfile(f.encode(), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl), ctypes.byref(by)):
            if n.value:
                out[f] = (n.value, ms.value, fl.value, by.value)
    return out


def configs_suite(steps=10, warmup=3, ids=None, cpu=True, graphs=True):
    """The other measured configurations of the backward path, each a full
    training step through the nn_engine API (synthetic inputs, seeds
    1000*config + {0: x, 1: weights, 2: labels}):
      1 LeNet-5 b64 (SGD lr 0.01, element clip 1.0)
      2 single conv backward x[128,64,56,56], W[128,64,3,3] p1, ReLU (dW + dX + db)
      3 MobileNetV2 inverted-residual stack b64 @112^2 + GAP + Linear 10 (SGD lr 0.01)
      4 UNet-base16 b8 @256^2, 4 levels, Dice on sigmoid, norm clip 1.0 + Adam lr 1e-3
    One JSON line per configuration: wall ms/step and img/s (no profiling in
    that timing), then per-family kernel ms/step with TFLOP/s or GB/s from a
    second, profiled pass (HIP events on the engine stream)."""
    from directcompute_torch_amd import nn_engine as nn
    lib = nn.lib
    T = lambda a, rg=False: nn.Tensor(np.ascontiguousarray(a, dtype=np.float32), requires_grad=rg, track=False)

    def he_conv(r, cout, cin, k):
        return T(r.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k)), True)

    def he_lin(r, fin, fout):
        return T(r.standard_normal((fin, fout)) * np.sqrt(2.0 / fin), True)

    def zeros(n, rg=True):
        return T(np.zeros(n), rg)

    def ones(n, rg=True):
        return T(np.ones(n), rg)

    def run_config(cid, name, batch, step, extra=None, mode="eager"):
        for _ in range(warmup):
            step()
        lib.SyncGPU()
        h0, m0 = ctypes.c_uint64(), ctypes.c_uint64()
        lib.GetPoolStats(ctypes.byref(h0), ctypes.byref(m0))
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        th = (time.perf_counter() - t0) / steps  # host issue time (queue not yet drained)
        lib.SyncGPU()
        dt = (time.perf_counter() - t0) / steps
        h1, m1 = ctypes.c_uint64(), ctypes.c_uint64()
        lib.GetPoolStats(ctypes.byref(h1), ctypes.byref(m1))
        pool = {"hits_per_step": (h1.value - h0.value) / steps, "misses_per_step": (m1.value - m0.value) / steps}
        lib.ResetProfile()
        if mode == "eager":   # a graph replay records no per-family events
            lib.SetProfiling(1)
            for _ in range(steps):
                step()
            lib.SyncGPU()
            lib.SetProfiling(0)
        fams = {}
        for f, (n, ms, fl, by) in _prof_all(lib).items():
            rec = {"launches_per_step": round(n / steps, 2), "ms_per_step": round(ms / steps, 4)}
            if fl:
                tf = fl / (ms * 1e-3) / 1e12
                rec.update({"TFLOP/s": round(tf, 2), "frac_mfma": round(tf / MFMA_FP32_PEAK_TFLOPS, 4)})
            elif by:
                gb = by / (ms * 1e-3) / 1e9
                rec.update({"GB/s": round(gb, 1), "frac_hbm": round(gb / HBM_PEAK_GBS, 4)})
            fams[f] = rec
        bwd = None
        allf = _prof_all(lib)
        if "conv_bwd" in allf:
            _, ms, fl, _ = allf["conv_bwd"]
            ms_g = sum(v[1] for k, v in allf.items() if k in ("conv_dw", "conv_dx"))
            tf = fl / (ms * 1e-3) / 1e12
            bwd = {"gflop_per_step": round(fl / steps / 1e9, 2), "ms_per_step": round(ms / steps, 4),
                   "TFLOP/s": round(tf, 2), "frac_mfma": round(tf / MFMA_FP32_PEAK_TFLOPS, 4),
                   "gemm_kernels_ms_per_step": round(ms_g / steps, 4),
                   "gemm_kernels_frac_mfma": round(fl / (ms_g * 1e-3) / 1e12 / MFMA_FP32_PEAK_TFLOPS, 4)}
        rec = {"suite": "configs", "config": cid, "mode": mode, "workload": name, "batch": batch,
               "ms_per_step": round(dt * 1e3, 4), "img_s": round(batch / dt, 1),
               "host_issue_ms_per_step": round(th * 1e3, 4),
               "conv_bwd": bwd, "pool": pool, "families": fams}
        if extra:
            rec.update(extra)
        if cpu and mode == "eager":
            nn.end_batch()
            rec["cpu_baseline"] = cpu_baseline_config(cid)
        print(json.dumps(rec), flush=True)
        log(f"[configs] {cid} {mode} {name}: {dt * 1e3:.3f} ms/step (host issue {th * 1e3:.3f}), {batch / dt:.0f} img/s"
            + (f"; conv-bwd {bwd['TFLOP/s']} TFLOP/s ({bwd['frac_mfma'] * 100:.1f}%)" if bwd else "")
            + f"; pool misses/step {pool['misses_per_step']:.1f} of {pool['hits_per_step'] + pool['misses_per_step']:.1f}")
        nn.end_batch()

    # 1 LeNet-5 b64
    def config1():
        r = np.random.default_rng(1001)
        P = [he_conv(r, 6, 1, 5), zeros(6), he_conv(r, 16, 6, 5), zeros(16),
             he_lin(r, 256, 120), zeros(120), he_lin(r, 120, 84), zeros(84), he_lin(r, 84, 10), zeros(10)]
        x = T(np.random.default_rng(1000).standard_normal((64, 1, 28, 28)))
        y = T(np.random.default_rng(1002).integers(0, 10, 64))
        opt = nn.SGD(P, lr=0.01)

        def lenet_step():
            opt.zero_grad()
            h = nn.maxpool2d(nn.conv2d(x, P[0], P[1], 1, 0, 1), 2, 2)
            h = nn.flatten(nn.maxpool2d(nn.conv2d(h, P[2], P[3], 1, 0, 1), 2, 2))
            h = nn.bias_relu(nn.matmul(h, P[4]), P[5])
            h = nn.bias_relu(nn.matmul(h, P[6]), P[7])
            loss = nn.softmax_ce(nn.add_bias(nn.matmul(h, P[8]), P[9]), y)
            loss.backward()
            opt.step(clip=1.0)
            nn.end_batch()
        run_config(1, "LeNet-5 b64 train step (SGD lr 0.01, clip 1.0)", 64, lenet_step)

        def lenet_fwd(xb):
            h = nn.maxpool2d(nn.conv2d(xb, P[0], P[1], 1, 0, 1), 2, 2)
            h = nn.flatten(nn.maxpool2d(nn.conv2d(h, P[2], P[3], 1, 0, 1), 2, 2))
            h = nn.bias_relu(nn.matmul(h, P[4]), P[5])
            h = nn.bias_relu(nn.matmul(h, P[6]), P[7])
            return nn.add_bias(nn.matmul(h, P[8]), P[9])
        if graphs:
            graph = nn.ComputeGraph()
            graph.trace(lenet_fwd, opt, x.sync(), y.sync(), P, clip=1.0)
            run_config(1, "LeNet-5 b64 train step (SGD lr 0.01, clip 1.0), replayed with ComputeGraph",
                       64, graph.replay, mode="graph")
            graph.release()

    # 2 single conv backward
    def config2():
        r = np.random.default_rng(2001)
        W, b = he_conv(r, 128, 64, 3), zeros(128)
        x2 = T(np.random.default_rng(2000).standard_normal((128, 64, 56, 56)), True)
        dy = np.random.default_rng(2002).standard_normal((128, 128, 56, 56)).astype(np.float32)
        gy = T(dy)

        def conv_step():
            W.grad = b.grad = x2.grad = None
            yv = nn.conv2d(x2, W, b, 1, 1, 1)
            yv.backward(gy)  # ConvBackwardFused masks dy with [y > 0]
            nn.end_batch()
        run_config(2, "single conv backward x[128,64,56,56] W[128,64,3,3] p1 ReLU: dW + dX + db",
                   128, conv_step, {"conv_bwd_gflop_algorithmic": round(2 * 2 * 128 * 64 * 9 * 128 * 56 * 56 / 1e9, 2)})

    # 3 MobileNetV2 inverted-residual stack b64 @112^2
    def config3():
        r = np.random.default_rng(3001)
        blocks = []
        for ci, co, s in [(16, 24, 2), (24, 24, 1), (24, 32, 2), (32, 32, 1), (32, 32, 1)]:
            h = ci * 6
            blocks.append(dict(ci=ci, co=co, s=s,
                               exp=(he_conv(r, h, ci, 1), zeros(h)),
                               bn1=(ones(h), zeros(h), zeros(h, False), ones(h, False)),
                               dw=(T(r.standard_normal((h, 1, 3, 3)) * np.sqrt(2.0 / 9), True), zeros(h)),
                               bn2=(ones(h), zeros(h), zeros(h, False), ones(h, False)),
                               proj=(he_conv(r, co, h, 1), zeros(co)),
                               bn3=(ones(co), zeros(co), zeros(co, False), ones(co, False))))
        fc = (he_lin(r, 32, 10), zeros(10))
        Pm = [fc[0], fc[1]]
        for bl in blocks:
            for k in ("exp", "dw", "proj"):
                Pm += list(bl[k])
            for k in ("bn1", "bn2", "bn3"):
                Pm += list(bl[k][:2])
        x3 = T(np.random.default_rng(3000).standard_normal((64, 16, 112, 112)))
        y3 = T(np.random.default_rng(3002).integers(0, 10, 64))
        opt3 = nn.SGD(Pm, lr=0.01)

        def mbv2_step():
            opt3.zero_grad()
            h = x3
            for bl in blocks:
                t = nn.relu6(nn.batchnorm2d(nn.conv2d(h, *bl["exp"], 1, 0, 0), *bl["bn1"]))
                t = nn.relu6(nn.batchnorm2d(nn.depthwise_conv2d(t, *bl["dw"], bl["s"], 1), *bl["bn2"]))
                t = nn.batchnorm2d(nn.conv2d(t, *bl["proj"], 1, 0, 0), *bl["bn3"])
                h = nn.add(t, h) if (bl["s"] == 1 and bl["ci"] == bl["co"]) else t
            loss = nn.softmax_ce(nn.add_bias(nn.matmul(nn.global_avg_pool2d(h), fc[0]), fc[1]), y3)
            loss.backward()
            opt3.step(clip=1e30)
            nn.end_batch()
        run_config(3, "MobileNetV2 IR stack b64 @112^2 (16-24 s2, 24-24, 24-32 s2, 32-32 x2; "
                      "expand x6, BN train, ReLU6, dw3x3) + GAP + Linear 10, SGD lr 0.01", 64, mbv2_step)

    # 4 UNet-base16 b8 @256^2
    def config4():
        r = np.random.default_rng(4001)
        U = {}

        def cbr_p(name, cin, cout):
            U[name] = (he_conv(r, cout, cin, 3), zeros(cout), ones(cout), zeros(cout),
                       zeros(cout, False), ones(cout, False))
        ch = [16, 32, 64, 128]
        prev = 3
        for i, c in enumerate(ch):
            cbr_p(f"e{i}a", prev, c)
            cbr_p(f"e{i}b", c, c)
            prev = c
        cbr_p("ba", prev, 256)
        cbr_p("bb", 256, 256)
        prev = 256
        for i in reversed(range(4)):
            cbr_p(f"d{i}a", prev + ch[i], ch[i])
            cbr_p(f"d{i}b", ch[i], ch[i])
            prev = ch[i]
        head = (he_conv(r, 1, 16, 1), zeros(1))
        Pu = list(head)
        for v in U.values():
            Pu += list(v[:4])
        x4 = T(np.random.default_rng(4000).random((8, 3, 256, 256)))
        m = (np.random.default_rng(4002).random((8, 1, 32, 32)) < 0.3).astype(np.float32)
        t4 = T(m.repeat(8, axis=2).repeat(8, axis=3))
        opt4 = nn.Adam(Pu, lr=1e-3)

        def cbr(h, name):
            w, bb, g, be, rm, rv = U[name]
            return nn.relu(nn.batchnorm2d(nn.conv2d(h, w, bb, 1, 1, 0), g, be, rm, rv))

        def unet_fwd(xb):
            h = xb
            skips = []
            for i in range(4):
                h = cbr(cbr(h, f"e{i}a"), f"e{i}b")
                skips.append(h)
                h = nn.maxpool2d(h, 2, 2)
            h = cbr(cbr(h, "ba"), "bb")
            for i in reversed(range(4)):
                h = nn.concat([nn.upsample2d(h, 2, 2), skips[i]])
                h = cbr(cbr(h, f"d{i}a"), f"d{i}b")
            return nn.sigmoid(nn.conv2d(h, head[0], head[1], 1, 0, 0))

        def unet_step():
            opt4.zero_grad()
            loss = nn.dice_loss(unet_fwd(x4), t4)
            loss.backward()
            nn.clip_grad_norm(Pu, 1.0)
            opt4.step(clip=1e30)
            nn.end_batch()
        name4 = "UNet-base16 b8 @256^2 (4 levels, conv3x3-BN-ReLU x2, Dice on sigmoid; norm clip 1.0 + Adam lr 1e-3)"
        run_config(4, name4, 8, unet_step)
        if graphs:
            graph = nn.ComputeGraph()
            graph.trace(unet_fwd, opt4, x4.sync(), t4.sync(), Pu, clip=1e30, loss_fn=nn.dice_loss,
                        max_norm=1.0)
            run_config(4, name4 + ", replayed with ComputeGraph", 8, graph.replay, mode="graph")
            graph.release()

    for cid, fn in ((1, config1), (2, config2), (3, config3), (4, config4)):
        if not ids or cid in ids:
            fn()


def copy_calibration(mib=256, reps=3):
    """Plain elementwise copy (torch's mul-by-one kernel) of `mib` MiB: each
    launch reads and writes exactly mib MiB, so its counter readings give the
    scale between rocprofv3's FETCH_SIZE / WRITE_SIZE and bytes."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"bytes_read": n * 4, "bytes_written": n * 4,
                                           "launches": reps}}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample", type=int, default=256)
    ap.add_argument("--suite", choices=["train", "memory", "configs"], default="train",
                    help="train: the AlexNet-224 b128 train step (default, one JSON line); "
                         "memory: the backward memory-bound kernels, one JSON line each; "
                         "configs: LeNet, single conv, MobileNetV2 stack, UNet steps, one line each")
    ap.add_argument("--configs", default="",
                    help="with --suite configs: comma-separated configuration numbers (default all)")
    ap.add_argument("--eager-only", action="store_true",
                    help="with --suite configs: skip the ComputeGraph replays (rocprofv3's kernel "
                         "tracing of graph capture crashed the process on this image)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of 256 MiB three times (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "the benchmark runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.suite == "memory":
        memory_suite()
        return
    if args.suite == "configs":
        ids = {int(v) for v in args.configs.split(",")} if args.configs else None
        configs_suite(steps=min(args.steps, 10), warmup=args.warmup, ids=ids,
                      cpu=not args.no_cpu_baseline, graphs=not args.eager_only)
        return

    from directcompute_torch_amd import nn_engine as nn
    lib = nn.lib
    log(f"[bench] device {nn._GPU_NAME}, VRAM {nn._VRAM_MB} MB")

    params = he_params(np.random.default_rng(SEED + 1))
    model = build_alexnet(nn, params)
    x = nn.Tensor(np.random.default_rng(SEED).standard_normal((BATCH, 3, 224, 224)).astype(np.float32), track=False)
    y = nn.Tensor(np.random.default_rng(SEED + 2).integers(0, 1000, BATCH).astype(np.float32), track=False)
    opt = nn.AdamW(model.parameters(), lr=1e-4, weight_decay=0.01)

    def step():
        opt.zero_grad()
        logits = model(x)
        loss = nn.softmax_ce(logits, y)
        loss.backward()
        opt.step(clip=1.0)
        nn.end_batch()
        return loss

    for _ in range(args.warmup):
        step()
    lib.SyncGPU()
    lib.ResetProfile()
    lib.SetProfileFilter(ROOFLINE_FAMILY.encode())
    lib.SetProfiling(1)
    h0, m0 = ctypes.c_uint64(), ctypes.c_uint64()
    lib.GetPoolStats(ctypes.byref(h0), ctypes.byref(m0))
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    lib.SyncGPU()
    t1 = time.perf_counter()
    h1, m1 = ctypes.c_uint64(), ctypes.c_uint64()
    lib.GetPoolStats(ctypes.byref(h1), ctypes.byref(m1))
    log(f"[bench] pool: {(m1.value - m0.value) / args.steps:.1f} misses of "
        f"{(h1.value + m1.value - h0.value - m0.value) / args.steps:.1f} buffer requests per step")
    lib.SetProfiling(0)

    dt = (t1 - t0) / args.steps
    img_s = BATCH / dt

    def prof(fam):
        n, ms, fl, by = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        if not lib.GetProfile(fam.encode(), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl), ctypes.byref(by)):
            return 0, 0.0, 0.0, 0.0
        return n.value, ms.value, fl.value, by.value

    fams = {ROOFLINE_FAMILY: prof(ROOFLINE_FAMILY)}
    # Breakdown pass (not timed): the other families over the same number of steps.
    lib.ResetProfile()
    lib.SetProfileFilter(b",".join(f.encode() for f in BREAKDOWN_FAMILIES))
    lib.SetProfiling(1)
    for _ in range(args.steps):
        step()
    lib.SyncGPU()
    lib.SetProfiling(0)
    lib.SetProfileFilter(None)
    fams.update({f: prof(f) for f in BREAKDOWN_FAMILIES})
    for f, (n, ms, fl, by) in fams.items():
        if n:
            extra = f"{fl / (ms * 1e-3) / 1e12:7.2f} TFLOP/s" if fl else f"{by / (ms * 1e-3) / 1e9:8.1f} GB/s"
            log(f"[bench] {f:12s} launches/step {n / args.steps:5.1f}  ms/step {ms / args.steps:8.3f}  {extra}")
    n_dw, ms_dw, fl_dw, _ = fams["conv_dw"]
    n_dx, ms_dx, fl_dx, _ = fams["conv_dx"]
    n_bwd, ms_bwd, fl_bwd, _ = fams["conv_bwd"]
    ms_gemm = ms_dw + ms_dx
    expect = conv_bwd_flops(BATCH) * args.steps
    for what, fl in (("conv-bwd calls", fl_bwd), ("conv-bwd GEMMs", fl_dw + fl_dx)):
        if abs(fl - expect) > 1e-6 * expect:
            log(f"[bench] WARNING {what} FLOP count {fl:.4e} != expected {expect:.4e}")
    achieved = fl_bwd / (ms_bwd * 1e-3) / 1e12 if ms_bwd > 0 else 0.0
    achieved_gemm = fl_bwd / (ms_gemm * 1e-3) / 1e12 if ms_gemm > 0 else 0.0
    log(f"[bench] {img_s:.1f} img/s, {dt * 1e3:.2f} ms/step; conv-bwd {achieved:.2f} TFLOP/s "
        f"({achieved / MFMA_FP32_PEAK_TFLOPS * 100:.1f}% of fp32 MFMA peak) over "
        f"{ms_bwd / args.steps:.3f} ms/step of ConvBackwardFused calls; their GEMM kernels alone "
        f"{achieved_gemm:.2f} TFLOP/s over {ms_gemm / args.steps:.3f} ms/step")

    # The same step with a fresh batch uploaded from (pageable) host memory
    # every step, as the reference's loop does.
    host_x = np.random.default_rng(SEED).standard_normal((BATCH, 3, 224, 224)).astype(np.float32)

    def step_upload():
        opt.zero_grad()
        xb = nn.Tensor(host_x, track=True)
        loss = nn.softmax_ce(model(xb), y)
        loss.backward()
        opt.step(clip=1.0)
        nn.end_batch()

    step_upload()
    lib.SyncGPU()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step_upload()
    lib.SyncGPU()
    dt_up = (time.perf_counter() - t0) / args.steps
    log(f"[bench] with a {host_x.nbytes / 2**20:.0f} MiB host batch uploaded every step: "
        f"{BATCH / dt_up:.1f} img/s, {dt_up * 1e3:.2f} ms/step")

    traffic, alg_bytes = measured_traffic()
    if traffic:
        traffic, alg_bytes = round(traffic), round(alg_bytes)
    out = {
        "metric": "train-step img/s, AlexNet-224 fp32 b128; conv-bwd TFLOP/s & % roofline",
        "value": round(img_s, 2),
        "unit": "img/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "value_upload_inclusive": round(BATCH / dt_up, 2),
        "ms_per_step_upload_inclusive": round(dt_up * 1e3, 4),
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": "AlexNet-224 full train step (fwd + bwd + AdamW lr=1e-4 wd=0.01 clip=1.0), "
                        "Linear 9216-4096-4096-1000, input [128,3,224,224] ~N(0,1), labels U{0..999}",
            "batch": BATCH,
            "conv_bwd_gflop_per_step": round(conv_bwd_flops(BATCH) / 1e9, 2),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "conv backward of all layers, each ConvBackwardFused call whole: G pass "
                      "k_to_nhwc (ReLU mask + NHWC transpose + bias partials, with the dX filter "
                      "re-layout as extra blocks; k_mask_pad for c1), dW k_igemm<LdGradKR,LdXTapKR> "
                      "(c1, C = 3: k_igemm<LdGPadRK,LdPsRK> on the stride-phase copy) + k_dw_final "
                      "(with the bias-gradient sum as extra blocks), dX k_igemm<LdDenseRK,LdPixRK> "
                      "(+ k_splitk_nchw4 when split)",
            "achieved": round(achieved, 3),
            "peak": MFMA_FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_FP32_PEAK_TFLOPS, 4),
            "gemm_kernels_achieved": round(achieved_gemm, 3),
            "gemm_kernels_frac": round(achieved_gemm / MFMA_FP32_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "traffic_unit": "HBM bytes per ConvBackwardFused call, all its kernels "
                            "(rocprofv3 FETCH_SIZE/WRITE_SIZE scaled by a copy kernel; "
                            "profiles/alexnet224_b128_conv_bwd_hbm_traffic.md)" if traffic else None,
            "algorithmic_bytes_per_call": alg_bytes,
            "calls_per_step": n_bwd / args.steps,
            "gemm_launches_per_step": (n_dw + n_dx) / args.steps,
            "ms_per_step": round(ms_bwd / args.steps, 4),
        },
    }
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU float64 oracle baseline ...")
        out["cpu_baseline"] = cpu_baseline(args.cpu_sample)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
