"""Benchmark: AlexNet-224 fp32 batch-128 training step on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]

One step = forward (5 conv + 3 maxpool + 3 linear), softmax-CE, the full
backward (conv dW/db/dX implicit-GEMM MFMA kernels, maxpool routing, linear
GEMMs, bias/ReLU gradients) and an AdamW update (lr 1e-4, wd 0.01, element
clip 1.0) of all 61.1 M parameters, through the drop-in ``nn_engine`` API.
Inputs are synthetic and already resident in device memory when the timed
region starts.  Prints ONE JSON line on stdout; diagnostics go to stderr.

Roofline object: the conv-backward implicit-GEMM kernels (dW and dX, all
layers of one step) timed with HIP events on the engine stream over the timed
region; achieved = algorithmic FLOPs (2*OC*C*k*k*B*OH*OW per dW and per dX;
c1 has no dX since the input needs no gradient) / summed kernel time.

cpu_baseline: the float64 NumPy oracle running the same train step on a
64-image sample on the host, timed on this machine.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
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


def cpu_baseline(sample=64):
    """Time the float64 oracle on the same train step for `sample` images."""
    from oracle import models as OM
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
    ap.add_argument("--cpu-sample", type=int, default=64)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of 256 MiB three times (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
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
    lib.SetProfiling(1)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    lib.SyncGPU()
    t1 = time.perf_counter()
    lib.SetProfiling(0)

    dt = (t1 - t0) / args.steps
    img_s = BATCH / dt

    def prof(fam):
        n, ms, fl, by = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        if not lib.GetProfile(fam.encode(), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl), ctypes.byref(by)):
            return 0, 0.0, 0.0, 0.0
        return n.value, ms.value, fl.value, by.value

    fams = {f: prof(f) for f in ("conv_dw", "conv_dx", "conv_fwd", "gemm", "maxpool_fwd", "maxpool_bwd", "adam")}
    for f, (n, ms, fl, by) in fams.items():
        if n:
            extra = f"{fl / (ms * 1e-3) / 1e12:7.2f} TFLOP/s" if fl else f"{by / (ms * 1e-3) / 1e9:8.1f} GB/s"
            log(f"[bench] {f:12s} launches/step {n / args.steps:5.1f}  ms/step {ms / args.steps:8.3f}  {extra}")
    n_dw, ms_dw, fl_dw, _ = fams["conv_dw"]
    n_dx, ms_dx, fl_dx, _ = fams["conv_dx"]
    ms_bwd = ms_dw + ms_dx
    fl_bwd = fl_dw + fl_dx
    expect = conv_bwd_flops(BATCH) * args.steps
    if abs(fl_bwd - expect) > 1e-6 * expect:
        log(f"[bench] WARNING conv-bwd FLOP count {fl_bwd:.4e} != expected {expect:.4e}")
    achieved = fl_bwd / (ms_bwd * 1e-3) / 1e12 if ms_bwd > 0 else 0.0
    log(f"[bench] {img_s:.1f} img/s, {dt * 1e3:.2f} ms/step; conv-bwd {achieved:.2f} TFLOP/s "
        f"({achieved / MFMA_FP32_PEAK_TFLOPS * 100:.1f}% of fp32 MFMA peak), "
        f"{ms_bwd / args.steps:.3f} ms/step in conv-bwd kernels")

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
            "kernel": "conv-backward implicit GEMM, all layers: dW k_igemm<LdGradKR,LdXTapKR> + k_dw_final, dX k_igemm<LdDenseRK,LdPixRK> (+ k_splitk_nchw when split)",
            "achieved": round(achieved, 3),
            "peak": MFMA_FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_FP32_PEAK_TFLOPS, 4),
            "traffic": None,
            "launches_per_step": (n_dw + n_dx) / args.steps,
            "kernel_ms_per_step": round(ms_bwd / args.steps, 4),
        },
    }
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU float64 oracle baseline ...")
        out["cpu_baseline"] = cpu_baseline(args.cpu_sample)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
