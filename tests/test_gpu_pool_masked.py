"""GPU parity of the max-pool backward that also makes the masked gradient of
the ReLU convolution under it (the conv_grad_reshape_relu step of
engine.cpp:816-835 done by the producer of dy, nn_maxpool_backward.hlsl:12-25
plus nn_conv_grad_reshape_relu.hlsl:21-39):

* MaxPoolBackwardFused over the output of a ReLU ConvForwardFused over fewer
  than 4 input channels (AlexNet c1, LeNet c1) returns dx as before and
  keeps, with it, the conv's masked G on the padded pixel grid that the
  conv's filter gradient reads, with the bias-gradient partials;
  ConvBackwardFused on that dx then runs no masking pass for it (other
  convolutions keep their transpose pass);
* dW and dX equal, bit for bit, those of the same call on an untagged copy
  of dx (same G); db (other partial sums) within 1e-6; all three against
  the float64 oracle within 1e-4;
* anything that writes y, dx or the pooled output in between (UpdateBuffer,
  a second gradient accumulated into dx) turns the shortcut off, and the
  results follow the written values."""
import ctypes

import numpy as np
import pytest

from oracle import kernels as K
from tests.helpers import TOL, download, he, rel_err, release, rng, upload
from tests.test_gpu_kernels import new, run

pytestmark = pytest.mark.gpu

# (B, C, H, W, OC, k, s, p, pool k): conv (ReLU) then max-pool (pool k, stride 2)
CASES = [
    (2, 3, 223, 223, 16, 11, 4, 2, 3),   # AlexNet c1 family: padded grid, 55x55 (odd) planes
    (2, 3, 59, 59, 8, 11, 4, 2, 3),      # padded grid, 14x14 planes: 2 pad columns past the blocks
    (2, 1, 28, 28, 6, 5, 1, 0, 2),       # LeNet c1: padded grid, 2x2 pool
    (2, 3, 30, 26, 12, 3, 1, 1, 3),      # odd, non-square planes (30x26 -> 14x12 windows)
    (1, 2, 7, 6, 4, 3, 1, 1, 3),         # two window columns (paired loads at their limit)
    (1, 3, 5, 4, 8, 3, 1, 1, 3),         # one window column (single loads)
    (2, 3, 13, 21, 5, 3, 1, 1, 2),       # 2x2 pool over odd planes
    (2, 16, 27, 27, 40, 5, 1, 2, 3),     # AlexNet c2 family: NHWC G, no shortcut
    (3, 6, 12, 12, 16, 5, 1, 0, 2),      # LeNet c2: NHWC G, no shortcut
]


def _launches(eng, fam):
    n, ms, fl, by = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    ok = eng.lib.GetProfile(fam.encode(), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl),
                            ctypes.byref(by))
    return int(n.value) if ok else 0


def _setup(eng, case, seed):
    B, C, H, W, OC, k, s, p, pk = case
    r = rng(seed)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    b = (0.1 * r.standard_normal(OC)).astype(np.float32)
    hx, hw, hb = upload(eng, x), upload(eng, w), upload(eng, b)
    pim = ctypes.c_void_p()
    hy = eng.lib.ConvForwardFused(hx, hw, hb, B, C, H, W, OC, k, k, s, p, 1, ctypes.byref(pim))
    assert hy, eng.last_error()
    OH, OW = K.conv_out_hw(H, W, k, s, p)
    y = download(eng, hy, (B, OC, OH, OW))
    pidx = ctypes.c_void_p()
    hz = eng.lib.MaxPoolForwardFused(hy, B, OC, OH, OW, pk, 2, ctypes.byref(pidx))
    assert hz, eng.last_error()
    PH, PW = (OH - pk) // 2 + 1, (OW - pk) // 2 + 1
    idx = download(eng, pidx.value, (B, OC, PH, PW)).view(np.uint32)
    dz = r.standard_normal((B, OC, PH, PW)).astype(np.float32)
    return dict(x=x, w=w, y=y, idx=idx, dz=dz, hx=hx, hw=hw, hb=hb, hy=hy, hz=hz, pim=pim.value,
                pidx=pidx.value, geo=(B, C, H, W, OC, k, s, p), pool=(PH, PW), r=r)


def _conv_bwd(eng, d, hdy, im2col, want_x=True):
    """ConvBackwardFused (dW, db and, with want_x, dX); returns the gradients
    and the number of masking passes (G_pad and NHWC G) the call ran."""
    B, C, H, W, OC, k, s, p = d["geo"]
    pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    eng.lib.ResetProfile()
    eng.lib.ConvBackwardFused(hdy, d["hy"], d["hx"], d["hw"], im2col, B, C, H, W, OC, k, k, s, p, 1,
                              int(want_x), 1, 1, ctypes.byref(pdf), ctypes.byref(pdb),
                              ctypes.byref(pdx))
    assert pdf.value and pdb.value and bool(pdx.value) == want_x, eng.last_error()
    out = (download(eng, pdf.value, d["w"].shape), download(eng, pdb.value, (OC,)),
           download(eng, pdx.value, d["x"].shape) if want_x else None)
    masking = _launches(eng, "conv_grad_nhwc")
    release(eng, pdf.value, pdb.value, pdx.value)
    return out, masking


def _check_oracle(got, dy, y, d, what):
    B, C, H, W, OC, k, s, p = d["geo"]
    dW_ref, db_ref, dX_ref = K.conv_backward(dy, y, d["x"], d["w"], s, p, 1)
    for name, g, ref in zip(("dW", "db", "dX"), got, (dW_ref, db_ref, dX_ref)):
        if g is None:
            continue
        e = rel_err(g, ref)
        assert e <= TOL, f"{what} {name}: {e:.3e}"


@pytest.mark.parametrize("want_x", [True, False], ids=["dX", "noDX"])
@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_pool_backward_makes_conv_g(eng, case, want_x):
    """The first layer of a network (AlexNet c1, LeNet c1) asks for no dX: with
    the padded-grid G made by the max-pool backward it runs no masking pass at
    all; with dX it still makes the NHWC G that dX reads."""
    B, C, H, W, OC, k, s, p, pk = case
    eng.lib.SetProfiling(1)
    try:
        d = _setup(eng, case, 4100 + sum(case))
        # fewer than 4 input channels (stride <= 4): the padded grid
        shortcut = C < 4 and s <= 4
        hdz = upload(eng, d["dz"])
        hdx = eng.lib.MaxPoolBackwardFused(hdz, d["pidx"], B, OC, *d["pool"], d["y"].size)
        assert hdx, eng.last_error()
        dx = download(eng, hdx, d["y"].shape)
        ref_dx = K.maxpool_backward(d["dz"], d["idx"], d["y"].size).reshape(d["y"].shape)
        assert rel_err(dx, ref_dx) <= 1e-6
        # an untagged copy of dx: 0 + dx, bit for bit
        hcopy = new(eng, dx.size)
        eng.lib.ClearBuffer(hcopy)
        run(eng, "grad_accum", [hdx], [hcopy], dx.size)
        assert np.array_equal(download(eng, hcopy, dx.shape), dx)
        fused, n_fused = _conv_bwd(eng, d, hdx, d["pim"], want_x)
        plain, n_plain = _conv_bwd(eng, d, hcopy, None, want_x)
        assert n_plain > 0
        assert n_fused == n_plain - int(shortcut), (n_fused, n_plain, shortcut)
        assert np.array_equal(fused[0], plain[0]), "dW differs from the unfused call"
        if want_x:
            assert np.array_equal(fused[2], plain[2]), "dX differs from the unfused call"
        assert rel_err(fused[1], plain[1]) <= 1e-6
        _check_oracle(fused, dx, d["y"], d, "fused")
        release(eng, hdz, hdx, hcopy, d["hx"], d["hw"], d["hb"], d["hy"], d["hz"])
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


@pytest.mark.parametrize("case", [CASES[0], CASES[2]], ids=["pool3", "pool2"])
@pytest.mark.parametrize("write", ["y", "dx", "pooled"])
def test_pool_g_shortcut_dropped_on_writes(eng, case, write):
    """A write to y (the conv output), to dx or to the pooled output between
    the forward and the conv backward turns the producer-made G off."""
    B, C, H, W, OC, k, s, p, pk = case
    eng.lib.SetProfiling(1)
    try:
        d = _setup(eng, case, 4200 + sum(case))
        y = d["y"]
        hdz = upload(eng, d["dz"])
        if write == "pooled":
            # The pooled values are what the masked backward reads; after a
            # write to them the max-pool backward makes dx only.
            z = download(eng, d["hz"], (B, OC) + d["pool"])
            eng.lib.UpdateBuffer(d["hz"], np.ascontiguousarray(-np.abs(z) - 1.0).ctypes.data_as(
                ctypes.POINTER(ctypes.c_float)))
        hdx = eng.lib.MaxPoolBackwardFused(hdz, d["pidx"], B, OC, *d["pool"], y.size)
        assert hdx, eng.last_error()
        dx = download(eng, hdx, y.shape)
        dy = dx
        if write == "y":
            # zero a third of the positive outputs: the mask must follow
            y2 = y.copy()
            pos = np.flatnonzero(y2 > 0)
            y2.flat[pos[::3]] = 0.0
            eng.lib.UpdateBuffer(d["hy"], y2.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
            y = y2
        elif write == "dx":
            extra = d["r"].standard_normal(y.shape).astype(np.float32)
            he_ = upload(eng, extra)
            run(eng, "grad_accum", [he_], [hdx], y.size)
            dy = download(eng, hdx, y.shape)
            release(eng, he_)
        got, masking = _conv_bwd(eng, d, hdx, d["pim"])
        assert masking > 0, "the masking pass must run after the write"
        _check_oracle(got, dy, y, d, write)
        release(eng, hdz, hdx, d["hx"], d["hw"], d["hb"], d["hy"], d["hz"])
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


def _random_cases(n, seed):
    """Seeded random ReLU convolutions over 1-3 input channels (strides 1-4:
    the padded-grid layout) followed by a 2x2 or 3x3 stride-2 max-pool: odd
    and even plane widths, pad-column counts 0-3, one-window-column planes."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k, s = int(r.integers(1, 8)), int(r.integers(1, 5))
        p = int(r.integers(0, k))
        H, W = int(r.integers(k, 40)), int(r.integers(k, 40))
        OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
        pk = int(r.choice([2, 3]))
        if OH < pk or OW < pk:
            continue
        out.append((int(r.integers(1, 4)), int(r.integers(1, 4)), H, W, int(r.integers(1, 40)),
                    k, s, p, pk))
    return out


RANDOM = _random_cases(16, 2718)


@pytest.mark.parametrize("case", RANDOM, ids=[str(c) for c in RANDOM])
def test_pool_backward_makes_conv_g_random(eng, case):
    test_pool_backward_makes_conv_g(eng, case, want_x=False)
