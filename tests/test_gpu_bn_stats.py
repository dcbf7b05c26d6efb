"""GPU parity of the batch-norm statistics left by a conv forward's GEMM, and
of the conv's NHWC G made by the batch-norm backward
(batchnorm_mean_var, nn_batchnorm_mean_var.hlsl:19-61, on the output of a
ConvForwardFused with no activation, engine.cpp:690-738):

* ConvForwardFused with actType 0 at stride 1 over 4 or more channels (pixel
  or pointwise GEMM; the split-K finish when K is split) writes y as before
  and keeps the per-channel sums of y and y*y;
  batchnorm_mean_var on y then only finishes them (family bn_stats_side,
  no pass over y), and mean, var and the running statistics agree with the
  same call on an untagged copy of y within 1e-6 (double sums in another
  order) and with the float64 oracle within 1e-5;
* depthwise_conv_forward (nn_depthwise_conv_forward.hlsl:24-50) through its
  band kernels (3x3 / 5x5, stride 1 / 2) leaves them too;
* layouts that do not leave statistics (C < 4, stride 2, ReLU) and
  any write to y in between (UpdateBuffer, a shader writing y) fall back to
  the statistics pass, and the results follow the written values;
* batchnorm_backward_dx over such a conv's output (when the conv's backward
  has a transpose pass: not pointwise) also writes the conv's NHWC G and
  bias-gradient partials; the BN dx and the conv's dW, db, dX are bit for
  bit those of the unfused chain, the conv backward runs no transpose pass,
  and a gradient accumulated into dx in between turns it off."""
import ctypes

import numpy as np
import pytest

from oracle import kernels as K
from tests.helpers import TOL, download, he, rel_err, release, rng, upload
from tests.test_gpu_kernels import fbits, new, run

pytestmark = pytest.mark.gpu

# (B, C, H, W, OC, k, s, p, act, side): side = the GEMM leaves the statistics
CASES = [
    (2, 16, 32, 32, 16, 3, 1, 1, 0, True),     # UNet level 0 shape (small)
    (2, 32, 17, 15, 32, 3, 1, 1, 0, True),     # ragged planes: a partial last column tile
    (3, 24, 9, 11, 72, 1, 1, 0, 0, True),      # pointwise expand (MobileNetV2)
    (1, 256, 8, 8, 256, 3, 1, 1, 0, True),     # deep channels, few pixels: split K (the finish leaves them)
    (2, 96, 14, 14, 24, 1, 1, 0, 0, True),     # pointwise project
    (1, 48, 20, 20, 20, 3, 1, 1, 0, True),     # OC not a multiple of the tile rows
    (2, 8, 12, 12, 136, 3, 1, 1, 0, True),     # OC past 128: two row blocks
    (1, 16, 5, 7, 12, 5, 1, 2, 0, True),       # 5x5, tiny planes (one column tile)
    (2, 3, 20, 20, 16, 3, 1, 1, 0, False),     # C < 4: stride-phase layout, no statistics
    (2, 16, 20, 20, 16, 3, 2, 1, 0, False),    # stride 2
    (2, 16, 20, 20, 16, 3, 1, 1, 1, False),    # ReLU
]


def _count(eng, fam):
    n, ms, fl, by = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    ok = eng.lib.GetProfile(fam.encode(), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl),
                            ctypes.byref(by))
    return int(n.value) if ok else 0


def _forward(eng, case, seed):
    B, C, H, W, OC, k, s, p, act, _ = case
    r = rng(seed)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    # a per-channel offset, so that the one-pass variance is exercised
    b = (0.5 + r.standard_normal(OC)).astype(np.float32)
    hx, hw, hb = upload(eng, x), upload(eng, w), upload(eng, b)
    hy = eng.lib.ConvForwardFused(hx, hw, hb, B, C, H, W, OC, k, k, s, p, act, None)
    assert hy, eng.last_error()
    OH, OW = K.conv_out_hw(H, W, k, s, p)
    y = download(eng, hy, (B, OC, OH, OW))
    assert rel_err(y, K.conv_forward(x, w, b, s, p, act)) <= TOL
    release(eng, hx, hw, hb)
    return hy, y, r


def _mean_var(eng, hy, shape, rm, rv, mom=0.1):
    """batchnorm_mean_var on hy; returns (mean, var, running mean, running
    var) and the launches of the two statistics families."""
    B, C, H, W = shape
    hmu, hvar, hrm, hrv = new(eng, C), new(eng, C), upload(eng, rm), upload(eng, rv)
    eng.lib.ResetProfile()
    run(eng, "batchnorm_mean_var", [hy], [hmu, hvar, hrm, hrv], B, C, H * W, 1, fbits(mom))
    out = [download(eng, h, (C,)) for h in (hmu, hvar, hrm, hrv)]
    fams = (_count(eng, "bn_stats_side"), _count(eng, "bn_stats"))
    release(eng, hmu, hvar, hrm, hrv)
    return out, fams


def _copy(eng, h, n):
    """An untagged copy of buffer h (0 + h, bit for bit)."""
    c = new(eng, n)
    eng.lib.ClearBuffer(c)
    run(eng, "grad_accum", [h], [c], n)
    return c


def _check_oracle(got, y, rm, rv, what, mom=0.1):
    ref = K.batchnorm_mean_var(y, rm, rv, mom, True)
    for name, g, rf in zip(("mean", "var", "running mean", "running var"), got, ref):
        assert rel_err(g, rf) <= 1e-5, f"{what} {name}: {rel_err(g, rf):.3e}"


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_conv_forward_leaves_bn_statistics(eng, case):
    side = case[-1]
    eng.lib.SetProfiling(1)
    try:
        hy, y, r = _forward(eng, case, 5100 + sum(case[:-1]))
        C = y.shape[1]
        rm = r.standard_normal(C).astype(np.float32)
        rv = (1.0 + r.random(C)).astype(np.float32)
        got, fams = _mean_var(eng, hy, y.shape, rm, rv)
        assert fams == ((1, 0) if side else (0, 1)), fams
        # the tag survives a read: a second call finishes the same sums
        again, fams2 = _mean_var(eng, hy, y.shape, rm, rv)
        assert fams2 == fams
        for a, b in zip(got, again):
            assert np.array_equal(a, b)
        hc = _copy(eng, hy, y.size)
        plain, pf = _mean_var(eng, hc, y.shape, rm, rv)
        assert pf == (0, 1)
        for name, a, b in zip(("mean", "var", "rm", "rv"), got, plain):
            assert rel_err(a, b) <= 1e-6, f"{name} vs the statistics pass: {rel_err(a, b):.3e}"
        _check_oracle(got, y, rm, rv, "side" if side else "pass")
        release(eng, hy, hc)
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


@pytest.mark.parametrize("write", ["update", "shader"])
def test_bn_statistics_dropped_on_writes(eng, write):
    """A write to y between the conv forward and batchnorm_mean_var turns the
    GEMM's statistics off; the statistics follow the written values."""
    case = CASES[0]
    eng.lib.SetProfiling(1)
    try:
        hy, y, r = _forward(eng, case, 5200)
        if write == "update":
            y = (2.0 * y + 1.0).astype(np.float32)
            eng.lib.UpdateBuffer(hy, np.ascontiguousarray(y).ctypes.data_as(
                ctypes.POINTER(ctypes.c_float)))
        else:
            extra = r.standard_normal(y.shape).astype(np.float32)
            he_ = upload(eng, extra)
            run(eng, "grad_accum", [he_], [hy], y.size)
            y = download(eng, hy, y.shape)
            release(eng, he_)
        C = y.shape[1]
        rm, rv = np.zeros(C, np.float32), np.ones(C, np.float32)
        got, fams = _mean_var(eng, hy, y.shape, rm, rv)
        assert fams == (0, 1), fams
        _check_oracle(got, y, rm, rv, write)
        release(eng, hy)
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


def test_bn_statistics_other_geometry(eng):
    """batchnorm_mean_var over y with another (N, C, S) view than the conv's
    output takes the statistics pass."""
    case = CASES[0]
    eng.lib.SetProfiling(1)
    try:
        hy, y, r = _forward(eng, case, 5300)
        B, C, H, W = y.shape
        view = (B * 2, C // 2, H, W)
        yv = y.reshape(view)
        rm, rv = np.zeros(view[1], np.float32), np.ones(view[1], np.float32)
        got, fams = _mean_var(eng, hy, view, rm, rv)
        assert fams == (0, 1), fams
        _check_oracle(got, yv, rm, rv, "view")
        release(eng, hy)
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


def _random_cases(n, seed):
    """Seeded stride-1, no-activation convolutions of 4-64 input channels
    (pixel GEMMs over the NHWC copy, or pointwise), 1-160 output channels."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k = int(r.choice([1, 3, 5]))
        p = 0 if k == 1 else int(r.integers(0, k // 2 + 1))
        H, W = int(r.integers(k, 40)), int(r.integers(k, 40))
        out.append((int(r.integers(1, 4)), int(r.integers(4, 65)), H, W, int(r.integers(1, 161)),
                    k, 1, p, 0, True))
    return out


RANDOM = _random_cases(12, 9001)


@pytest.mark.parametrize("case", RANDOM, ids=[str(c) for c in RANDOM])
def test_conv_forward_leaves_bn_statistics_random(eng, case):
    test_conv_forward_leaves_bn_statistics(eng, case)


# (B, C, H, W, k, s, p): depthwise convolutions on the band kernels
DW_CASES = [
    (2, 24, 28, 28, 3, 1, 1),     # MobileNetV2 dw 3x3 s1
    (2, 16, 29, 31, 3, 2, 1),     # stride 2, odd planes
    (1, 8, 17, 12, 5, 1, 2),      # 5x5
    (3, 5, 9, 9, 5, 2, 2),        # 5x5 stride 2, ragged channels
    (2, 4, 57, 6, 3, 1, 0),       # tall narrow planes, no padding
]


@pytest.mark.parametrize("case", DW_CASES, ids=[str(c) for c in DW_CASES])
def test_depthwise_forward_leaves_bn_statistics(eng, case):
    B, C, H, W, k, s, p = case
    r = rng(5400 + sum(case))
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    f = (r.standard_normal((C, 1, k, k)) / k).astype(np.float32)
    fb = (0.5 + r.standard_normal(C)).astype(np.float32)
    OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    hx, hf, hfb, hy = upload(eng, x), upload(eng, f), upload(eng, fb), new(eng, B * C * OH * OW)
    eng.lib.SetProfiling(1)
    try:
        run(eng, "depthwise_conv_forward", [hx, hf, hfb], [hy], B, C, H, W, k, k, s, p, OH)
        y = download(eng, hy, (B, C, OH, OW))
        assert rel_err(y, K.depthwise_forward(x, f, fb, s, p)) <= 1e-5
        rm = r.standard_normal(C).astype(np.float32)
        rv = (1.0 + r.random(C)).astype(np.float32)
        got, fams = _mean_var(eng, hy, y.shape, rm, rv)
        assert fams == (1, 0), fams
        hc = _copy(eng, hy, y.size)
        plain, pf = _mean_var(eng, hc, y.shape, rm, rv)
        assert pf == (0, 1)
        for name, a, b in zip(("mean", "var", "rm", "rv"), got, plain):
            assert rel_err(a, b) <= 1e-6, f"{name} vs the statistics pass: {rel_err(a, b):.3e}"
        _check_oracle(got, y, rm, rv, "depthwise")
        # a second forward into the same output replaces the statistics
        x2 = (2.0 * x - 1.0).astype(np.float32)
        eng.lib.UpdateBuffer(hx, x2.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        run(eng, "depthwise_conv_forward", [hx, hf, hfb], [hy], B, C, H, W, k, k, s, p, OH)
        y2 = download(eng, hy, (B, C, OH, OW))
        got2, fams2 = _mean_var(eng, hy, y.shape, rm, rv)
        assert fams2 == (1, 0)
        _check_oracle(got2, y2, rm, rv, "depthwise again")
        release(eng, hx, hf, hfb, hy, hc)
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


# (B, C, H, W, OC, k, s, p): conv (no activation) -> batch norm; the BN
# backward makes the conv's NHWC G when the conv's backward has a transpose pass
BNG_CASES = [
    (2, 16, 24, 24, 16, 3, 1, 1),     # UNet level 0 shape (16 channels: 128-pixel blocks)
    (2, 32, 13, 17, 48, 3, 1, 1),     # 48 channels: 64-pixel blocks, ragged planes
    (1, 8, 9, 9, 6, 5, 1, 2),         # OC not a multiple of 4 (padded G rows)
    (2, 24, 10, 10, 40, 3, 2, 1),     # stride 2 (the forward leaves no statistics: plain BN dx)
    (2, 24, 8, 8, 36, 1, 1, 0),       # pointwise: no transpose pass, plain BN dx
]


def _bn_chain(eng, case, seed, write_dx=False):
    """conv -> BN forward -> BN backward -> ConvBackwardFused; returns what the
    fused chain and the same calls on untagged copies give, and the launch
    counts of the conv backward's transpose passes."""
    B, C, H, W, OC, k, s, p = case
    r = rng(seed)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    b = (0.5 + r.standard_normal(OC)).astype(np.float32)
    hx, hw, hb = upload(eng, x), upload(eng, w), upload(eng, b)
    pim = ctypes.c_void_p()
    hy = eng.lib.ConvForwardFused(hx, hw, hb, B, C, H, W, OC, k, k, s, p, 0, ctypes.byref(pim))
    assert hy, eng.last_error()
    OH, OW = K.conv_out_hw(H, W, k, s, p)
    y = download(eng, hy, (B, OC, OH, OW))
    S_ = OH * OW
    gamma = (1.0 + 0.2 * r.standard_normal(OC)).astype(np.float32)
    hg = upload(eng, gamma)
    hmu, hvar = new(eng, OC), new(eng, OC)
    hrm, hrv = upload(eng, np.zeros(OC, np.float32)), upload(eng, np.ones(OC, np.float32))
    run(eng, "batchnorm_mean_var", [hy], [hmu, hvar, hrm, hrv], B, OC, S_, 1, fbits(0.1))
    dz = r.standard_normal(y.shape).astype(np.float32)
    hdz = upload(eng, dz)
    eps = 1e-5
    hdg, hdb = new(eng, OC), new(eng, OC)
    run(eng, "batchnorm_backward_reduce", [hy, hdz, hmu, hvar], [hdg, hdb], B, OC, S_, fbits(eps))
    out = {}
    yc = _copy(eng, hy, y.size)
    for name, hin in (("fused", hy), ("plain", yc)):
        hdx = new(eng, y.size)
        run(eng, "batchnorm_backward_dx", [hin, hdz, hmu, hvar, hg, hdg, hdb], [hdx], B, OC, S_,
            fbits(eps))
        if write_dx and name == "fused":
            extra = r.standard_normal(y.shape).astype(np.float32)
            he_ = upload(eng, extra)
            run(eng, "grad_accum", [he_], [hdx], y.size)
            release(eng, he_)
        dx_bn = download(eng, hdx, y.shape)
        # the conv backward on this dx; a ConvBackwardFused consumes the
        # forward's copy of x, so the plain call gets a second forward's
        pim_b = pim
        if name == "plain":
            pim_b = ctypes.c_void_p()
            hy2 = eng.lib.ConvForwardFused(hx, hw, hb, B, C, H, W, OC, k, k, s, p, 0,
                                           ctypes.byref(pim_b))
            assert hy2, eng.last_error()
            release(eng, hy2)
        pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        eng.lib.ResetProfile()
        eng.lib.ConvBackwardFused(hdx, None, hx, hw, pim_b.value, B, C, H, W, OC, k, k, s, p, 0, 1,
                                  1, 1, ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
        assert pdf.value and pdb.value and pdx.value, eng.last_error()
        out[name] = dict(dx_bn=dx_bn, dW=download(eng, pdf.value, w.shape),
                         db=download(eng, pdb.value, (OC,)), dX=download(eng, pdx.value, x.shape),
                         passes=_count(eng, "nhwc") + _count(eng, "conv_grad_nhwc"))
        release(eng, hdx, pdf.value, pdb.value, pdx.value)
    release(eng, hx, hw, hb, hy, yc, hg, hmu, hvar, hrm, hrv, hdz, hdg, hdb)
    return out, dict(x=x, w=w, y=y, s=s, p=p)


def _check_conv_oracle(f, d, s, p):
    """dW, dX against the float64 oracle within TOL; db, a sum over every
    pixel of a batch norm's dx (zero up to round-off, as that dx sums to
    zero per channel), within 1e-5 of the channel's sum of |dx|."""
    dW_r, db_r, dX_r = K.conv_backward(f["dx_bn"], d["y"], d["x"], d["w"], s, p, 0)
    for name, ref in (("dW", dW_r), ("dX", dX_r)):
        assert rel_err(f[name], ref) <= TOL, f"{name}: {rel_err(f[name], ref):.3e}"
    scale = np.abs(f["dx_bn"].astype(np.float64)).sum(axis=(0, 2, 3))
    assert np.all(np.abs(f["db"] - db_r) <= 1e-5 * scale), "db"


@pytest.mark.parametrize("case", BNG_CASES, ids=[str(c) for c in BNG_CASES])
def test_bn_backward_makes_conv_g(eng, case):
    B, C, H, W, OC, k, s, p = case
    fused_g = s == 1 and k > 1
    eng.lib.SetProfiling(1)
    try:
        out, d = _bn_chain(eng, case, 5500 + sum(case))
        f, q = out["fused"], out["plain"]
        assert np.array_equal(f["dx_bn"], q["dx_bn"]), "BN dx differs from the plain kernel"
        for name in ("dW", "dX", "db"):
            assert np.array_equal(f[name], q[name]), f"{name} differs from the unfused chain"
        if fused_g:
            assert f["passes"] == 0 and q["passes"] > 0, (f["passes"], q["passes"])
        else:
            assert f["passes"] == q["passes"]
        _check_conv_oracle(f, d, s, p)
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


def test_bn_backward_g_dropped_on_write(eng):
    """A gradient accumulated into the BN's dx before the conv backward turns
    the G off; the conv backward follows the accumulated values."""
    case = BNG_CASES[0]
    B, C, H, W, OC, k, s, p = case
    eng.lib.SetProfiling(1)
    try:
        out, d = _bn_chain(eng, case, 5600, write_dx=True)
        f = out["fused"]
        assert f["passes"] > 0
        _check_conv_oracle(f, d, s, p)
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


def _bn_forward(eng, hx, shape, hg, hb, eps=1e-5):
    B, C, H, W = shape
    hmu, hvar = new(eng, C), new(eng, C)
    hrm, hrv = upload(eng, np.zeros(C, np.float32)), upload(eng, np.ones(C, np.float32))
    run(eng, "batchnorm_mean_var", [hx], [hmu, hvar, hrm, hrv], B, C, H * W, 1, fbits(0.1))
    hz = new(eng, B * C * H * W)
    run(eng, "batchnorm_forward", [hx, hmu, hvar, hg, hb], [hz], B, C, H * W, fbits(eps))
    release(eng, hmu, hvar, hrm, hrv)
    return hz


@pytest.mark.parametrize("act", ["relu", "relu6"])
def test_bn_forward_stores_next_activation(eng, act):
    """batchnorm_forward also stores the activation that followed the same
    layer (gamma buffer) last time; that relu / relu6 call then adopts it
    (no launch) with the bits its own kernel gives.  A write to z in
    between, another activation or another element count runs the kernel."""
    B, C, H, W = 2, 12, 10, 8
    r = rng(5700 + len(act))
    n = B * C * H * W
    x = (2.0 * r.standard_normal((B, C, H, W))).astype(np.float32)
    gamma = (1.0 + r.standard_normal(C)).astype(np.float32)
    beta = (3.0 * r.standard_normal(C)).astype(np.float32)
    hx, hg, hb = upload(eng, x), upload(eng, gamma), upload(eng, beta)
    ref_fn = K.relu if act == "relu" else K.relu6
    cb = () if act == "relu" else (n,)
    eng.lib.SetProfiling(1)
    try:
        outs = []
        for rnd in range(3):
            hz = _bn_forward(eng, hx, x.shape, hg, hb)
            z = download(eng, hz, x.shape)
            ha = new(eng, n)
            eng.lib.ResetProfile()
            run(eng, act, [hz], [ha], *cb)
            launches = _count(eng, act)
            a = download(eng, ha, x.shape)
            assert np.array_equal(a, ref_fn(z).astype(np.float32)), rnd
            outs.append((a, launches))
            release(eng, hz, ha)
        assert outs[0][1] == 1 and outs[1][1] == 0 and outs[2][1] == 0, [o[1] for o in outs]
        assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][0], outs[2][0])
        # a write to z in between: the kernel runs on the written values
        hz = _bn_forward(eng, hx, x.shape, hg, hb)
        z2 = (download(eng, hz, x.shape) - 1.0).astype(np.float32)
        eng.lib.UpdateBuffer(hz, z2.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        ha = new(eng, n)
        eng.lib.ResetProfile()
        run(eng, act, [hz], [ha], *cb)
        assert _count(eng, act) == 1
        assert np.array_equal(download(eng, ha, x.shape), ref_fn(z2).astype(np.float32))
        release(eng, hz, ha)
        # the other activation on this layer's output: its own kernel
        other = "relu6" if act == "relu" else "relu"
        hz = _bn_forward(eng, hx, x.shape, hg, hb)
        z = download(eng, hz, x.shape)
        ha = new(eng, n)
        eng.lib.ResetProfile()
        run(eng, other, [hz], [ha], *(() if other == "relu" else (n,)))
        assert _count(eng, other) == 1
        ofn = K.relu if other == "relu" else K.relu6
        assert np.array_equal(download(eng, ha, x.shape), ofn(z).astype(np.float32))
        release(eng, hz, ha)
        # `act` again (the kernel: the layer stored the other one), then an
        # output of other elements than the stored one: the kernel
        hz = _bn_forward(eng, hx, x.shape, hg, hb)
        ha = new(eng, n)
        eng.lib.ResetProfile()
        run(eng, act, [hz], [ha], *cb)
        assert _count(eng, act) == 1
        release(eng, hz, ha)
        hz = _bn_forward(eng, hx, x.shape, hg, hb)
        z = download(eng, hz, x.shape).reshape(-1)
        ha = new(eng, n - 8 if act == "relu" else n)
        eng.lib.ResetProfile()
        run(eng, act, [hz], [ha], *(() if act == "relu" else (n - 8,)))
        assert _count(eng, act) == 1
        a = download(eng, ha, (n - 8 if act == "relu" else n,))
        assert np.array_equal(a[:n - 8], ref_fn(z)[:n - 8].astype(np.float32))
        release(eng, hz, ha)
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()
        release(eng, hx, hg, hb)


def _bn_act_setup(eng, seed, act):
    """conv (no activation) -> batchnorm_mean_var -> batchnorm_forward -> act;
    returns the handles the backward needs."""
    B, C, H, W, OC, k, s, p = 2, 16, 12, 12, 24, 3, 1, 1
    r = rng(seed)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    b = (0.5 + r.standard_normal(OC)).astype(np.float32)
    hx, hw, hb = upload(eng, x), upload(eng, w), upload(eng, b)
    hy = eng.lib.ConvForwardFused(hx, hw, hb, B, C, H, W, OC, k, k, s, p, 0, None)
    assert hy, eng.last_error()
    shape = (B, OC, H, W)
    n = B * OC * H * W
    gamma = (1.0 + 0.3 * r.standard_normal(OC)).astype(np.float32)
    beta = r.standard_normal(OC).astype(np.float32)
    hg, hbe = upload(eng, gamma), upload(eng, beta)
    hmu, hvar = new(eng, OC), new(eng, OC)
    hrm, hrv = upload(eng, np.zeros(OC, np.float32)), upload(eng, np.ones(OC, np.float32))
    run(eng, "batchnorm_mean_var", [hy], [hmu, hvar, hrm, hrv], B, OC, H * W, 1, fbits(0.1))
    hz = new(eng, n)
    run(eng, "batchnorm_forward", [hy, hmu, hvar, hg, hbe], [hz], B, OC, H * W, fbits(1e-5))
    ha = new(eng, n)
    run(eng, act, [hz], [ha], *(() if act == "relu" else (n,)))
    da = r.standard_normal(shape).astype(np.float32)
    hda = upload(eng, da)
    release(eng, hx, hw, hb, hrm, hrv, hbe)
    return dict(hy=hy, hz=hz, ha=ha, hda=hda, hg=hg, hmu=hmu, hvar=hvar, shape=shape, n=n, r=r)


def _act_grad_reduce(eng, h, act, z_handle, eps=1e-5, write=None):
    """act's backward into a new dz, then batchnorm_backward_reduce over
    (y, dz); returns dz, dgamma, dbeta and the reduce families' launches."""
    B, OC, H, W = h["shape"]
    n = h["n"]
    hdz = new(eng, n)
    run(eng, act + "_grad", [h["hda"], z_handle], [hdz], n)
    if write == "dz":
        he_ = upload(eng, h["r"].standard_normal(h["shape"]).astype(np.float32))
        run(eng, "grad_accum", [he_], [hdz], n)
        release(eng, he_)
    hdg, hdb = new(eng, OC), new(eng, OC)
    eng.lib.ResetProfile()
    run(eng, "batchnorm_backward_reduce", [h["hy"], hdz, h["hmu"], h["hvar"]], [hdg, hdb], B, OC,
        H * W, fbits(eps))
    fams = (_count(eng, "bn_bwd_reduce_side"), _count(eng, "bn_bwd_reduce"))
    out = (download(eng, hdz, h["shape"]), download(eng, hdg, (OC,)), download(eng, hdb, (OC,)))
    release(eng, hdz, hdg, hdb)
    return out, fams


@pytest.mark.parametrize("act", ["relu", "relu6"])
def test_act_grad_makes_bn_reduce_sums(eng, act):
    """relu_grad / relu6_grad over a batch norm's output also leaves the sums
    of that batch norm's backward reduce over (y, dz): dz, dgamma and dbeta
    are bit for bit those of the unfused calls, and the reduce reads no
    tensor; a write to y, the statistics or dz in between, or another eps,
    runs the reduce pass."""
    eng.lib.SetProfiling(1)
    try:
        h = _bn_act_setup(eng, 5800 + len(act), act)
        zc = _copy(eng, h["hz"], h["n"])  # untagged: the unfused calls
        (dz, dg, db), fams = _act_grad_reduce(eng, h, act, h["hz"])
        assert fams == (1, 0), fams
        (dz_p, dg_p, db_p), fams_p = _act_grad_reduce(eng, h, act, zc)
        assert fams_p == (0, 1), fams_p
        assert np.array_equal(dz, dz_p) and np.array_equal(dg, dg_p) and np.array_equal(db, db_p)
        # against the oracle
        y = download(eng, h["hy"], h["shape"])
        mu, var = download(eng, h["hmu"], (h["shape"][1],)), download(eng, h["hvar"], (h["shape"][1],))
        dg_r, db_r = K.batchnorm_backward_reduce(y, dz, mu, var, 1e-5)
        assert rel_err(dg, dg_r) <= TOL and rel_err(db, db_r) <= TOL
        # another eps: the pass
        _, fams_e = _act_grad_reduce(eng, h, act, h["hz"], eps=1e-3)
        assert fams_e == (0, 1), fams_e
        # a gradient accumulated into dz in between: the pass, on the new dz
        (dz_w, dg_w, db_w), fams_w = _act_grad_reduce(eng, h, act, h["hz"], write="dz")
        assert fams_w == (0, 1), fams_w
        dg_r, db_r = K.batchnorm_backward_reduce(y, dz_w, mu, var, 1e-5)
        assert rel_err(dg_w, dg_r) <= TOL and rel_err(db_w, db_r) <= TOL
        # a write to the batch statistics: no sums (the reduce reads the new ones)
        var2 = (var * 2.0 + 0.5).astype(np.float32)
        eng.lib.UpdateBuffer(h["hvar"], var2.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        (dz_v, dg_v, db_v), fams_v = _act_grad_reduce(eng, h, act, h["hz"])
        assert fams_v == (0, 1), fams_v
        dg_r, db_r = K.batchnorm_backward_reduce(y, dz_v, mu, var2, 1e-5)
        assert rel_err(dg_v, dg_r) <= TOL and rel_err(db_v, db_r) <= TOL
        release(eng, zc, h["hy"], h["hz"], h["ha"], h["hda"], h["hg"], h["hmu"], h["hvar"])
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()


def test_act_grad_bn_sums_dropped_on_x_write(eng):
    """A write to the batch norm's input y after its forward: the activation's
    backward leaves no sums and the reduce follows the written y."""
    eng.lib.SetProfiling(1)
    try:
        h = _bn_act_setup(eng, 5900, "relu")
        y = download(eng, h["hy"], h["shape"])
        y2 = (y + 0.25).astype(np.float32)
        eng.lib.UpdateBuffer(h["hy"], y2.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        (dz, dg, db), fams = _act_grad_reduce(eng, h, "relu", h["hz"])
        assert fams == (0, 1), fams
        mu = download(eng, h["hmu"], (h["shape"][1],))
        var = download(eng, h["hvar"], (h["shape"][1],))
        dg_r, db_r = K.batchnorm_backward_reduce(y2, dz, mu, var, 1e-5)
        assert rel_err(dg, dg_r) <= TOL and rel_err(db, db_r) <= TOL
        release(eng, h["hy"], h["hz"], h["ha"], h["hda"], h["hg"], h["hmu"], h["hvar"])
    finally:
        eng.lib.SetProfiling(0)
        eng.lib.ResetProfile()
