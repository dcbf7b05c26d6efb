"""GPU parity of the MFMA implicit-GEMM path against the float64 oracle:
MatMulAlloc (all flag combinations, split-K and ragged shapes), ConvForwardFused
and ConvBackwardFused (dW, fused db, dX; ReLU mask; strides, padding, kernel
sizes, channel counts that take the chunked and the flat K layouts)."""
import ctypes

import numpy as np
import pytest

from oracle import kernels as K
from tests import workloads as WL
from tests.helpers import TOL, download, he, rel_err, release, rng, upload

pytestmark = pytest.mark.gpu


GEMM_SHAPES = [
    (1, 1, 1), (5, 7, 3), (16, 16, 16), (17, 33, 65), (63, 64, 65), (64, 128, 64),
    (127, 129, 130), (128, 1000, 10), (6, 18432, 25), (16, 32768, 27), (200, 300, 100),
    (128, 9216, 256), (300, 40, 500),
]


@pytest.mark.parametrize("M,Kd,N", GEMM_SHAPES)
@pytest.mark.parametrize("flags", [0, 1, 2, 3])
def test_matmul_alloc(eng, M, Kd, N, flags):
    r = rng(1000 + M * 7 + Kd * 3 + N + flags)
    a = r.standard_normal((M, Kd)).astype(np.float32)
    b = r.standard_normal((Kd, N)).astype(np.float32)
    a_raw = a.T.copy() if flags & 1 else a
    b_raw = b.T.copy() if flags & 2 else b
    ha, hb = upload(eng, a_raw), upload(eng, b_raw)
    hc = eng.lib.MatMulAlloc(ha, hb, M, Kd, N, flags)
    assert hc, eng.last_error()
    c = download(eng, hc, (M, N))
    ref = K.matmul(a_raw, b_raw, M, Kd, N, flags)
    release(eng, ha, hb, hc)
    assert rel_err(c, ref) <= TOL


def _random_gemm_cases(n, seed):
    r = rng(seed)
    return [(int(r.integers(1, 300)), int(r.integers(1, 700)), int(r.integers(1, 300)), int(r.integers(0, 4)))
            for _ in range(n)]


RANDOM_GEMM_CASES = _random_gemm_cases(24, 4242)


@pytest.mark.parametrize("M,Kd,N,flags", RANDOM_GEMM_CASES)
def test_matmul_alloc_random_shapes(eng, M, Kd, N, flags):
    """MatMulAlloc on seeded random shapes and transpose flags (ragged tiles,
    padded operand copies, split-K and the small-GEMM tiles)."""
    test_matmul_alloc(eng, M, Kd, N, flags)


CONV_CASES = [
    # B, C, H, W, OC, k, s, p, act
    (2, 3, 9, 8, 4, 3, 1, 1, 1),
    (2, 1, 28, 28, 6, 5, 1, 0, 0),        # LeNet c1
    (3, 6, 12, 12, 16, 5, 1, 0, 1),       # LeNet c2
    (2, 16, 13, 11, 32, 3, 1, 1, 1),      # chunked K (C % 16 == 0)
    (2, 48, 10, 10, 16, 3, 1, 1, 1),      # UNet-style concat channels
    (2, 3, 35, 35, 64, 11, 4, 2, 1),      # AlexNet c1 geometry (small)
    (2, 64, 13, 13, 192, 5, 1, 2, 1),     # AlexNet c2 geometry
    (1, 32, 16, 16, 24, 1, 1, 0, 0),      # 1x1 (MobileNet project)
    (2, 24, 15, 15, 144, 1, 1, 0, 0),     # 1x1 expand, OC % 16 == 0 (dW with taps as rows)
    (2, 16, 12, 12, 96, 1, 1, 0, 1),      # 1x1 expand x6 (dW with taps as rows)
    (2, 3, 10, 11, 40, 1, 1, 0, 1),       # 1x1, C = 3 padded to 4 (dW with taps as rows)
    (2, 3, 64, 64, 16, 3, 1, 1, 1),       # one dW tile: many split-K slices
    (2, 2, 7, 9, 8, 3, 2, 1, 1),          # C = 2 (channel-packed x), stride 2
    (2, 3, 30, 30, 8, 5, 2, 1, 1),        # C = 3, padded width 32 (16-byte stores of the packed copy)
    (2, 16, 14, 14, 20, 3, 2, 1, 1),      # stride 2, OC not multiple of 16
    (2, 17, 9, 9, 33, 3, 2, 0, 2),        # tanh act: no derivative applied (reference quirk)
    (1, 8, 7, 7, 8, 3, 3, 1, 0),          # stride 3
    (2, 192, 6, 6, 256, 3, 1, 1, 1),      # deep channels
    # narrow dW tiles 32 columns wide (144 / 288 / 72 taps x channels)
    (2, 16, 24, 24, 16, 3, 1, 1, 1),
    (2, 32, 20, 20, 16, 3, 1, 1, 0),
    (2, 8, 18, 18, 12, 3, 1, 1, 1),       # 72 columns: the last 32-wide tile partly past N
    # C < 4 and stride <= 4: the stride-phase copy (padded pixel grid)
    (2, 1, 19, 21, 6, 3, 3, 1, 1),        # C = 1, stride 3, OW 7 -> 8 padded columns
    (2, 2, 17, 29, 12, 4, 4, 0, 0),       # even k, stride 4, no activation
    (2, 3, 9, 9, 5, 1, 2, 0, 1),          # 1x1, stride 2
    (2, 3, 224, 224, 64, 11, 4, 2, 1),    # AlexNet c1 at full resolution
    # C < 4 and stride > 4: the channel-packed copy
    (2, 3, 23, 23, 8, 7, 5, 2, 1),
    (1, 1, 20, 22, 4, 6, 6, 0, 1),
    # pointwise (1x1, planes of a multiple of 4 pixels, C >= 4): NCHW GEMMs in place
    (2, 96, 14, 14, 24, 1, 1, 0, 0),      # MobileNetV2 project
    (4, 5, 8, 8, 7, 1, 1, 0, 0),          # ragged channel counts (padded K)
    (2, 144, 28, 28, 32, 1, 1, 0, 2),     # tanh: no derivative, so no mask
    (8, 16, 56, 56, 96, 1, 1, 0, 0),      # expand at a MobileNet plane size (split-K dW)
    (2, 40, 6, 6, 130, 1, 1, 0, 0),       # db column at a tile edge (N = 41), OC past 128
    (3, 5, 8, 12, 40, 1, 1, 0, 0),        # expand: input channels (+ db row) as the dW rows
]


def _conv_case(eng, B, C, H, W, OC, k, s, p, act, want=(1, 1, 1), seed=0, keep=True):
    r = rng(2000 + seed + B + C * 3 + H * 5 + OC * 7 + k + s + p)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    b = (0.1 * r.standard_normal(OC)).astype(np.float32)
    hx, hw, hb = upload(eng, x), upload(eng, w), upload(eng, b)
    pim = ctypes.c_void_p()
    hy = eng.lib.ConvForwardFused(hx, hw, hb, B, C, H, W, OC, k, k, s, p, act,
                                  ctypes.byref(pim) if keep else None)
    assert hy, eng.last_error()
    OH, OW = K.conv_out_hw(H, W, k, s, p)
    y = download(eng, hy, (B, OC, OH, OW))
    y_ref = K.conv_forward(x, w, b, s, p, act)
    assert rel_err(y, y_ref) <= TOL, "forward"
    dy = r.standard_normal(y.shape).astype(np.float32)
    hdy = upload(eng, dy)
    pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    eng.lib.ConvBackwardFused(hdy, hy if act == 1 else None, hx, hw, pim.value, B, C, H, W, OC, k, k,
                              s, p, act, want[0], want[1], want[2],
                              ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
    # Mask from the device's own forward output (exact same y the kernel saw).
    dW_ref, db_ref, dX_ref = K.conv_backward(dy, y, x, w, s, p, act, need_x=want[0],
                                             need_w=want[1], need_b=want[2])
    out = {}
    if want[1]:
        assert pdf.value, eng.last_error()
        out["dW"] = (download(eng, pdf.value, w.shape), dW_ref)
    else:
        assert not pdf.value
    if want[2]:
        assert pdb.value, eng.last_error()
        out["db"] = (download(eng, pdb.value, (OC,)), db_ref)
    else:
        assert not pdb.value
    if want[0]:
        assert pdx.value, eng.last_error()
        out["dX"] = (download(eng, pdx.value, x.shape), dX_ref)
    else:
        assert not pdx.value
    release(eng, hx, hw, hb, hy, hdy, pdf.value, pdb.value, pdx.value)
    for name, (got, ref) in out.items():
        assert rel_err(got, ref) <= TOL, f"{name}: {rel_err(got, ref):.3e}"


@pytest.mark.parametrize("case", CONV_CASES, ids=[str(c) for c in CONV_CASES])
def test_conv_forward_backward(eng, case):
    _conv_case(eng, *case)


def _random_conv_cases(n, seed):
    """Seeded random geometries (each layout: stride-phase, channel-packed,
    pointwise, NHWC at every stride / pad / kernel size up to 7, ragged
    channel counts, tiny and odd planes)."""
    r = rng(seed)
    out = []
    while len(out) < n:
        k = int(r.integers(1, 8))
        s = int(r.integers(1, 6))
        p = int(r.integers(0, k))
        H, W = int(r.integers(k, 24)), int(r.integers(k, 24))
        if (H + 2 * p - k) // s + 1 < 1 or (W + 2 * p - k) // s + 1 < 1:
            continue
        out.append((int(r.integers(1, 4)), int(r.integers(1, 41)), H, W, int(r.integers(1, 70)),
                    k, s, p, int(r.integers(0, 3))))
    return out


RANDOM_CONV_CASES = _random_conv_cases(40, 31337)


@pytest.mark.parametrize("case", RANDOM_CONV_CASES, ids=[str(c) for c in RANDOM_CONV_CASES])
def test_conv_random_geometries(eng, case):
    """Forward, dW, db and dX against the float64 oracle on seeded random
    geometries (with and without the forward's channel-innermost copy)."""
    _conv_case(eng, *case, seed=23, keep=bool(case[0] % 2))


def _random_special_cases(n, seed, pointwise):
    """Seeded geometries of the two special layouts: inputs of 1-3 channels
    (stride-phase copy for strides up to 4, channel-packed above) with
    kernels up to 11, or pointwise 1x1 stride-1 layers on NCHW planes."""
    r = rng(seed)
    out = []
    while len(out) < n:
        if pointwise:
            k, s, p, C = 1, 1, 0, int(r.integers(1, 65))
            H, W = int(r.integers(1, 31)), int(r.integers(1, 31))
        else:
            k, s = int(r.integers(1, 12)), int(r.integers(1, 6))
            p, C = int(r.integers(0, k)), int(r.integers(1, 4))
            H, W = int(r.integers(k, 40)), int(r.integers(k, 40))
        if (H + 2 * p - k) // s + 1 < 1 or (W + 2 * p - k) // s + 1 < 1:
            continue
        out.append((int(r.integers(1, 4)), C, H, W, int(r.integers(1, 97)), k, s, p,
                    int(r.integers(0, 3))))
    return out


SPECIAL_CASES = _random_special_cases(16, 4242, False) + _random_special_cases(16, 2424, True)


@pytest.mark.parametrize("case", SPECIAL_CASES, ids=[str(c) for c in SPECIAL_CASES])
def test_conv_random_special_layouts(eng, case):
    """The stride-phase / channel-packed (C < 4) and pointwise layouts on
    seeded random geometries: forward, dW, db and dX against the float64
    oracle."""
    _conv_case(eng, *case, seed=29, keep=bool(case[1] % 2))


def _random_tile_rule_cases(n, seed):
    """Seeded geometries for the padding-aware tile choices: pointwise layers
    with 16-32 input (or output) channels and 33-160 on the other side (the
    short-K products on unsplit 32-row tiles), and 3x3 layers over 8-32
    channels with at most 32 output channels (the dW on 32-column narrow
    tiles when 64 columns would pad its taps x channels)."""
    r = rng(seed)
    out = []
    for i in range(n):
        B = int(r.integers(1, 4))
        H, W = 4 * int(r.integers(2, 9)), int(r.integers(4, 17))
        if i % 2 == 0:
            few, many = int(r.choice([16, 24, 32])), int(r.integers(33, 161))
            C, OC = (few, many) if r.integers(0, 2) else (many, few)
            out.append((B, C, H, W, OC, 1, 1, 0, int(r.integers(0, 2))))
        else:
            C, OC = int(r.choice([8, 16, 24, 32])), int(r.integers(1, 33))
            out.append((B, C, H, W, OC, 3, 1, 1, int(r.integers(0, 2))))
    return out


TILE_RULE_CASES = _random_tile_rule_cases(12, 777)


@pytest.mark.parametrize("case", TILE_RULE_CASES, ids=[str(c) for c in TILE_RULE_CASES])
def test_conv_tile_rule_geometries(eng, case):
    """Forward, dW, db and dX against the float64 oracle where the tile
    choice depends on the padding of the rows and columns."""
    _conv_case(eng, *case, seed=31, keep=True)


PHASE_CASES = [
    # stride >= 3: dX as s*s sub-pixel phases, each a GEMM over its own taps
    (2, 24, 20, 19, 32, 2, 3, 0, 1),      # k < s: phases without taps (zero planes)
    (1, 64, 30, 30, 48, 5, 3, 2, 1),      # 2 or 1 taps per phase row, odd phase planes
    (2, 16, 33, 31, 20, 7, 4, 3, 0),      # no activation, ragged plane widths
    (1, 40, 17, 17, 64, 4, 4, 0, 1),      # k == s: one tap per phase
    (2, 8, 26, 23, 16, 1, 3, 0, 1),       # 1x1 stride 3: one live phase
    (1, 32, 45, 45, 96, 11, 4, 2, 1),     # AlexNet c1 shape over 32 channels
]


@pytest.mark.parametrize("case", PHASE_CASES, ids=[str(c) for c in PHASE_CASES])
def test_conv_dx_stride_phases(eng, case):
    """Strided dX by sub-pixel phases against the float64 oracle (with and
    without the forward's channel-innermost copy)."""
    _conv_case(eng, *case, seed=37, keep=True)
    _conv_case(eng, *case, want=(1, 0, 0), seed=38, keep=False)


@pytest.mark.parametrize("case", [(2, 3, 35, 35, 64, 11, 4, 2, 1), (2, 1, 12, 10, 6, 5, 1, 2, 1),
                                  (2, 2, 20, 20, 4, 6, 5, 1, 1), (2, 16, 9, 9, 8, 3, 1, 1, 1)],
                         ids=str)
def test_conv_backward_rebuilds_x_copy(eng, case):
    """Without the forward's handle the backward builds its own copy of x
    (stride-phase or channel-packed for C < 4, NHWC otherwise)."""
    _conv_case(eng, *case, seed=5, keep=False)


@pytest.mark.parametrize("want", [(0, 1, 1), (1, 0, 0), (0, 0, 1), (1, 1, 0)])
def test_conv_backward_subsets(eng, want):
    _conv_case(eng, 2, 16, 10, 10, 32, 3, 1, 1, 1, want=want, seed=11)


@pytest.mark.parametrize("want", [(0, 1, 1), (1, 0, 0), (0, 0, 1), (1, 1, 0), (0, 1, 0)])
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("C,OC", [(32, 48), (8, 72)], ids=["c32_48", "expand_8_72"])
def test_pointwise_conv_backward_subsets(eng, want, act, C, OC):
    """Pointwise layers: every gradient subset, without (NCHW GEMMs in place;
    db alone goes through the general path) and with the ReLU mask (the
    general path, building the NHWC copy the forward did not keep); 8 -> 72
    channels puts the input channels on the dW product's rows."""
    _conv_case(eng, 2, C, 12, 12, OC, 1, 1, 0, act, want=want, seed=13)
    _conv_case(eng, 2, C, 12, 12, OC, 1, 1, 0, act, want=want, seed=14, keep=False)


PS_CASES = [
    (2, 3, 35, 35, 64, 11, 4, 2, 1),      # AlexNet c1 geometry (OW 8, no pad columns)
    (2, 3, 23, 21, 72, 5, 2, 1, 1),       # OW 10 -> 12 padded columns
    (2, 2, 7, 7, 6, 3, 2, 0, 1),          # OW 3: rows of fewer than 4 elements
    (2, 1, 12, 12, 40, 3, 1, 1, 1),       # 9 taps, 40 channels: taps as the dW rows
    (1, 3, 6, 5, 8, 5, 1, 2, 0),          # no activation (no mask)
]


@pytest.mark.parametrize("case", PS_CASES)
@pytest.mark.parametrize("want", [(0, 1, 1), (0, 1, 0), (0, 0, 1), (1, 1, 1), (1, 0, 1), (1, 1, 0)])
def test_stride_phase_backward_subsets(eng, case, want):
    """Fewer than 4 input channels (stride-phase copy): every gradient subset,
    with the masked gradient on the padded pixel grid (dW, db) and the NHWC
    gradient (dX; db when dW is not wanted)."""
    _conv_case(eng, *case, want=want, seed=17)


def test_stride_phase_relu_mask_nan_keeps_grad(eng):
    """The masked gradient on the padded pixel grid (stride-phase dW and db):
    y <= 0 zeroes it, a NaN y keeps it (nn_conv_grad_reshape_relu.hlsl:36), in
    the last quad of an output row as in the others."""
    B, C, H, W, OC, k, s, p = 2, 3, 23, 21, 8, 5, 2, 1
    OH, OW = K.conv_out_hw(H, W, k, s, p)
    r = rng(78)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    y = r.standard_normal((B, OC, OH, OW)).astype(np.float32)
    y[0, 0, 0, 0] = np.nan
    y[1, 2, 3, OW - 1] = np.nan
    y[0, 1, 1, OW - 2] = 0.0
    dy = r.standard_normal(y.shape).astype(np.float32)
    hs = [upload(eng, a) for a in (x, w, y, dy)]
    pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    eng.lib.ConvBackwardFused(hs[3], hs[2], hs[0], hs[1], None, B, C, H, W, OC, k, k, s, p, 1, 0, 1, 1,
                              ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
    assert pdf.value and pdb.value and not pdx.value, eng.last_error()
    dW_ref, db_ref, _ = K.conv_backward(dy, y, x, w, s, p, 1, need_x=0)
    got = (download(eng, pdf.value, w.shape), download(eng, pdb.value, (OC,)))
    release(eng, *hs, pdf.value, pdb.value)
    for g, ref in zip(got, (dW_ref, db_ref)):
        assert np.isfinite(g).all() == np.isfinite(ref).all()
        assert rel_err(g, ref) <= TOL


def test_conv_backward_relu_mask_nan_keeps_grad(eng):
    """y <= 0 zeroes the gradient; NaN in y keeps it (nn_conv_grad_reshape_relu.hlsl:36)."""
    B, C, H, W, OC, k = 1, 16, 6, 6, 16, 3
    r = rng(77)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    y = r.standard_normal((B, OC, H, W)).astype(np.float32)
    y[0, 0, 0, 0] = np.nan
    y[0, 1, 1, 1] = 0.0
    dy = r.standard_normal(y.shape).astype(np.float32)
    hs = [upload(eng, a) for a in (x, w, y, dy)]
    pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    eng.lib.ConvBackwardFused(hs[3], hs[2], hs[0], hs[1], None, B, C, H, W, OC, k, k, 1, 1, 1, 1, 1, 1,
                              ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
    dW_ref, db_ref, dX_ref = K.conv_backward(dy, y, x, w, 1, 1, 1)
    got = (download(eng, pdf.value, w.shape), download(eng, pdb.value, (OC,)), download(eng, pdx.value, x.shape))
    release(eng, *hs, pdf.value, pdb.value, pdx.value)
    for g, ref in zip(got, (dW_ref, db_ref, dX_ref)):
        assert rel_err(g, ref) <= TOL


def test_conv_backward_consumes_im2col_handle(eng):
    """ConvBackwardFused releases the im2col handle it is given (engine.cpp:877)."""
    h = upload(eng, np.zeros(16, np.float32))
    x = upload(eng, np.ones((1, 1, 4, 4), np.float32))
    w = upload(eng, np.ones((1, 1, 3, 3), np.float32))
    dy = upload(eng, np.ones((1, 1, 2, 2), np.float32))
    pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    eng.lib.ClearLastError()
    eng.lib.ConvBackwardFused(dy, None, x, w, h, 1, 1, 4, 4, 1, 3, 3, 1, 0, 0, 1, 1, 1,
                              ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
    assert eng.last_error() == ""
    eng.lib.ReleaseBuffer(h)  # second release of a consumed handle is rejected, not a crash
    assert "not live" in eng.last_error()
    release(eng, x, w, dy, pdf.value, pdb.value, pdx.value)


def test_single_conv_full_size_sampled(eng):
    """The single-conv workload at full size (x[128,64,56,56], W[128,64,3,3],
    s1 p1, ReLU mask): every dW/db entry and a sample of dX pixels are checked
    against float64 sums computed directly over the full batch."""
    B, C, H, W, OC, k = 128, 64, 56, 56, 128, 3
    r = rng(2 * 1000)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    b = np.zeros(OC, np.float32)
    hx, hw, hb = upload(eng, x), upload(eng, w), upload(eng, b)
    hy = eng.lib.ConvForwardFused(hx, hw, hb, B, C, H, W, OC, k, k, 1, 1, 1, None)
    assert hy, eng.last_error()
    y = download(eng, hy, (B, OC, H, W))
    oc_fwd = np.sort(rng(2 * 1000 + 1).choice(OC, 8, replace=False))
    _audit_forward(y, _fwd_ref_sampled(x, w, b, 1, 1, oc_fwd), oc_fwd, "single conv")
    dy = r.standard_normal(y.shape).astype(np.float32)
    hdy = upload(eng, dy)
    pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    eng.lib.ConvBackwardFused(hdy, hy, hx, hw, None, B, C, H, W, OC, k, k, 1, 1, 1, 1, 1, 1,
                              ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
    dW = download(eng, pdf.value, w.shape)
    db = download(eng, pdb.value, (OC,))
    dX = download(eng, pdx.value, x.shape)
    release(eng, hx, hw, hb, hy, hdy, pdf.value, pdb.value, pdx.value)
    G = np.where(y <= 0, 0.0, dy.astype(np.float64))
    # db: full check
    assert rel_err(db, G.sum(axis=(0, 2, 3))) <= TOL
    # dW: all (oc, c, kh, kw) via per-tap batched contractions over the full batch
    xp = np.zeros((B, C, H + 2, W + 2), np.float32)
    xp[:, :, 1:-1, 1:-1] = x
    dW_ref = np.empty(w.shape, np.float64)
    Gf = G.transpose(1, 0, 2, 3).reshape(OC, -1)
    for kh in range(k):
        for kw in range(k):
            xs = xp[:, :, kh:kh + H, kw:kw + W].transpose(1, 0, 2, 3).reshape(C, -1).astype(np.float64)
            dW_ref[:, :, kh, kw] = Gf @ xs.T
    assert rel_err(dW, dW_ref) <= TOL
    # dX: 64 sampled (b, ih, iw) pixels, all channels:
    # dX[b, c, ih, iw] = sum_{oc,kh,kw} W[oc, c, kh, kw] * G[b, oc, ih + 1 - kh, iw + 1 - kw]
    Gp = np.zeros((B, OC, H + 2, W + 2))
    Gp[:, :, 1:-1, 1:-1] = G
    w64 = w.astype(np.float64)
    ref_s, got_s = [], []
    for _ in range(64):
        bb, ih, iw = int(r.integers(B)), int(r.integers(H)), int(r.integers(W))
        acc = np.zeros(C)
        for kh in range(k):
            for kw in range(k):
                acc += w64[:, :, kh, kw].T @ Gp[bb, :, ih + 2 - kh, iw + 2 - kw]
        ref_s.append(acc)
        got_s.append(dX[bb, :, ih, iw])
    assert rel_err(np.array(got_s), np.array(ref_s)) <= TOL


def _fwd_ref_sampled(x, w, b, s, p, oc_sel):
    """Pre-activations z[b, oc, oh, ow] of the selected output channels over
    the whole batch, in float64: one contraction over the channels per tap."""
    B, C, H, W = x.shape
    k = w.shape[2]
    OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    xp = np.zeros((B, C, H + 2 * p, W + 2 * p), np.float32)
    xp[:, :, p:p + H, p:p + W] = x
    ws = w[oc_sel].astype(np.float64)
    z = np.zeros((B, len(oc_sel), OH, OW)) + b[oc_sel].astype(np.float64).reshape(1, -1, 1, 1)
    for kh in range(k):
        for kw in range(k):
            xs = xp[:, :, kh:kh + s * (OH - 1) + 1:s, kw:kw + s * (OW - 1) + 1:s].astype(np.float64)
            z += np.einsum("oc,bchw->bohw", ws[:, :, kh, kw], xs, optimize=True)
    return z


def _audit_forward(y, z_sel, oc_sel, what):
    """The device's ReLU forward on the sampled channels against the float64
    pre-activations: the decisions the backward adopts (y > 0) may disagree
    with z > 0 only at near-ties, and the positive outputs match z."""
    a = WL.DecisionAudit()
    a.relu("pos", z_sel, y[:, oc_sel], dev_is_output=True)
    print(f"  {what} forward, {len(oc_sel)} sampled channels: {a.check(1e-5, 1e-5)}", flush=True)


def _dw_ref_taps(G, x, k, s, p, oc_sel):
    """dW[oc, c, kh, kw] for the selected output channels: one float64
    contraction over the whole batch per tap."""
    B, C, H, W = x.shape
    OH, OW = G.shape[2], G.shape[3]
    xp = np.zeros((B, C, H + 2 * p, W + 2 * p), np.float32)
    xp[:, :, p:p + H, p:p + W] = x
    Gf = G[:, oc_sel].transpose(1, 0, 2, 3).reshape(len(oc_sel), -1)
    out = np.empty((len(oc_sel), C, k, k))
    for kh in range(k):
        for kw in range(k):
            xs = xp[:, :, kh:kh + s * (OH - 1) + 1:s, kw:kw + s * (OW - 1) + 1:s]
            out[:, :, kh, kw] = Gf @ xs.transpose(1, 0, 2, 3).reshape(C, -1).astype(np.float64).T
    return out


@pytest.mark.parametrize("layer", ["c1", "c2"])
def test_alexnet_b128_conv_backward_full_size(eng, layer):
    """The AlexNet-224 batch-128 c1 (x[128,3,224,224], W[64,3,11,11], s4 p2:
    the stride-phase dW) and c2 (x[128,64,27,27], W[192,64,5,5], s1 p2)
    backward at the timed size, ReLU mask from the device's forward: db and
    dW of every (c1) or 24 sampled (c2) output channels against float64
    contractions over the full batch, and for c2 32 sampled dX pixels."""
    B, C, H, OC, k, s, p = (128, 3, 224, 64, 11, 4, 2) if layer == "c1" else (128, 64, 27, 192, 5, 1, 2)
    print(f"alexnet b128 {layer} backward", flush=True)
    r = rng(5 * 1000 + k)
    x = r.standard_normal((B, C, H, H)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    b = np.zeros(OC, np.float32)
    hx, hw, hb = upload(eng, x), upload(eng, w), upload(eng, b)
    pim = ctypes.c_void_p()
    hy = eng.lib.ConvForwardFused(hx, hw, hb, B, C, H, H, OC, k, k, s, p, 1, ctypes.byref(pim))
    assert hy, eng.last_error()
    OH, OW = K.conv_out_hw(H, H, k, s, p)
    y = download(eng, hy, (B, OC, OH, OW))
    oc_fwd = np.sort(rng(5 * 1000 + k + 1).choice(OC, 16, replace=False))
    _audit_forward(y, _fwd_ref_sampled(x, w, b, s, p, oc_fwd), oc_fwd, f"alexnet b128 {layer}")
    dy = r.standard_normal(y.shape).astype(np.float32)
    hdy = upload(eng, dy)
    want_x = 0 if layer == "c1" else 1
    pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    eng.lib.ConvBackwardFused(hdy, hy, hx, hw, pim.value, B, C, H, H, OC, k, k, s, p, 1, want_x, 1, 1,
                              ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
    assert pdf.value and pdb.value, eng.last_error()
    dW = download(eng, pdf.value, w.shape)
    db = download(eng, pdb.value, (OC,))
    dX = download(eng, pdx.value, x.shape) if want_x else None
    release(eng, hx, hw, hb, hy, hdy, pdf.value, pdb.value, pdx.value)
    G = np.where(y <= 0, 0.0, dy.astype(np.float64))
    assert rel_err(db, G.sum(axis=(0, 2, 3))) <= TOL
    oc_sel = np.arange(OC) if layer == "c1" else np.sort(r.choice(OC, 24, replace=False))
    assert rel_err(dW[oc_sel], _dw_ref_taps(G, x, k, s, p, oc_sel)) <= TOL
    if want_x:
        Gp = np.zeros((B, OC, OH + 2 * p, OW + 2 * p))
        Gp[:, :, p:p + OH, p:p + OW] = G
        w64 = w.astype(np.float64)
        ref_s, got_s = [], []
        for _ in range(32):
            bb, ih, iw = int(r.integers(B)), int(r.integers(H)), int(r.integers(H))
            acc = np.zeros(C)
            for kh in range(k):
                for kw in range(k):   # stride 1: oh = ih + p - kh
                    acc += w64[:, :, kh, kw].T @ Gp[bb, :, ih + 2 * p - kh, iw + 2 * p - kw]
            ref_s.append(acc)
            got_s.append(dX[bb, :, ih, iw])
        assert rel_err(np.array(got_s), np.array(ref_s)) <= TOL


TILE_CFGS = [f"{mt},{nt},{kt},{sp}" for mt in (64, 128) for nt in (64, 128) for kt in (16, 32)
             for sp in (1, 3)] + [f"{mt},{nt},16,{sp}" for mt, nt in ((256, 128), (128, 256)) for sp in (1, 3)]


@pytest.mark.parametrize("cfg", TILE_CFGS)
def test_forced_tile_configs(eng, monkeypatch, cfg):
    """Every tile shape, K depth and split-K count (forced through the
    DCE_TUNE_* overrides, split-K included for the forward and dX GEMMs that
    the heuristic never splits) gives the oracle's result."""
    for var in ("DCE_TUNE_FWD", "DCE_TUNE_DW", "DCE_TUNE_DX", "DCE_TUNE_GEMM"):
        monkeypatch.setenv(var, cfg)
    _conv_case(eng, 2, 16, 14, 14, 20, 3, 2, 1, 1)   # stride 2, OC not a multiple of 16
    _conv_case(eng, 2, 48, 10, 10, 16, 3, 1, 1, 1)   # stride 1
    _conv_case(eng, 2, 3, 23, 21, 72, 5, 2, 1, 1)    # C = 3: stride-phase dW (75 taps, OC 72)
    for flags in range(4):
        test_matmul_alloc(eng, 127, 129, 130, flags)
        test_matmul_alloc(eng, 5, 7, 3, flags)


NARROW_CFGS = [(f"{mt},{nt},16,{sp}", f"{mt},{nd},16,{sp}") for mt in (16, 32)
               for nt, nd in ((128, 64), (256, 128)) for sp in (1, 3)]


@pytest.mark.parametrize("pix_cfg,dense_cfg", NARROW_CFGS, ids=[c[0] for c in NARROW_CFGS])
def test_forced_narrow_tiles(eng, monkeypatch, pix_cfg, dense_cfg):
    """The narrow 16- and 32-row tiles (1x4 wave grid, A operand staged by a
    subset of the threads), forced on every GEMM family, including output
    channel counts above the tile height (several M tiles) and split-K."""
    for var in ("DCE_TUNE_FWD", "DCE_TUNE_DX"):
        monkeypatch.setenv(var, pix_cfg)
    for var in ("DCE_TUNE_DW", "DCE_TUNE_GEMM"):
        monkeypatch.setenv(var, dense_cfg)
    _conv_case(eng, 2, 16, 14, 14, 20, 3, 2, 1, 1)   # stride 2, OC 20 (two 16-row tiles)
    _conv_case(eng, 2, 48, 10, 10, 16, 3, 1, 1, 1)   # stride 1, C 48 (dX: three 16-row tiles)
    _conv_case(eng, 3, 3, 17, 19, 8, 5, 1, 2, 1)     # C = 3 padded to 4, OC 8
    for flags in range(4):
        test_matmul_alloc(eng, 37, 129, 70, flags)
        test_matmul_alloc(eng, 5, 7, 3, flags)


KSPLIT_CFGS = [f"{mt},{nt},64,{sp}" for mt in (16, 32) for nt in (64, 128) for sp in (1, 3)]


@pytest.mark.parametrize("cfg", KSPLIT_CFGS)
def test_forced_narrow_ksplit_tiles(eng, monkeypatch, cfg):
    """The narrow tiles whose four waves split each 64-deep K tile and add
    their partial tiles at the end, forced on the dW and dense GEMMs (the
    pixel GEMMs take K tiles of 16 only), with several M tiles and split-K."""
    for var in ("DCE_TUNE_DW", "DCE_TUNE_GEMM"):
        monkeypatch.setenv(var, cfg)
    _conv_case(eng, 2, 16, 14, 14, 20, 3, 2, 1, 1)   # OC 20: two 16-row tiles
    _conv_case(eng, 2, 48, 10, 10, 40, 3, 1, 1, 1)   # OC 40: two 32-row tiles
    _conv_case(eng, 3, 3, 17, 19, 8, 5, 1, 2, 1)     # C = 3 padded to 4, OC 8
    for flags in range(4):
        test_matmul_alloc(eng, 37, 129, 70, flags)
        test_matmul_alloc(eng, 5, 7, 3, flags)


def test_linear_tile_order(eng, monkeypatch):
    """DCE_XCD=0 (plain tile order) gives the same results as the default
    XCD-contiguous order."""
    monkeypatch.setenv("DCE_XCD", "0")
    _conv_case(eng, 2, 64, 13, 13, 192, 5, 1, 2, 1)
    test_matmul_alloc(eng, 200, 300, 100, 0)


# ------------------------------------------- direct valid convolutions
def _run_shader(eng, name, srvs, uavs, cb):
    import struct
    sa = (ctypes.c_void_p * len(srvs))(*srvs)
    ua = (ctypes.c_void_p * len(uavs))(*uavs)
    th = (ctypes.c_uint * 3)(1, 1, 1)
    words = [struct.unpack("I", struct.pack("I", v))[0] for v in cb]
    cba = (ctypes.c_uint * len(words))(*words)
    eng.lib.ClearLastError()
    eng.lib.RunShader(name.encode(), sa, len(srvs), ua, len(uavs), th,
                      ctypes.cast(cba, ctypes.c_void_p), 4 * len(words))
    assert eng.last_error() == "", eng.last_error()


TILED_GPU = [(4, 16, 20, 20, 24, 3), (2, 3, 30, 26, 8, 5), (3, 20, 16, 16, 12, 1), (2, 7, 13, 11, 5, 4),
             (16, 32, 28, 28, 64, 3)]


@pytest.mark.parametrize("B,C,H,W,OC,k", TILED_GPU)
def test_tiled_conv_shaders(eng, B, C, H, W, OC, k):
    """conv_forward_tiled, conv_backprop_filters_tiled and
    conv_backprop_input_fused (nn_engine.py:148; valid convolution, stride 1,
    no padding) through RunShader with the reference's constant layout, on
    the implicit-GEMM core (generic, stride-phase C < 4 and pointwise k = 1
    layouts), against the float64 oracle: act 0 / ReLU / tanh forward, the
    filter gradient (its dB slot left untouched, as the shader never writes
    it) and the input gradient times the previous ReLU / tanh derivative."""
    print(f"tiled conv shaders B{B} C{C} {H}x{W} OC{OC} k{k}", flush=True)
    r = rng(B * 1000 + C * 37 + k)
    OH, OW = H - k + 1, W - k + 1
    geo = (B, C, H, W, OC, k, OH, OW)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    w = he(r, (OC, C, k, k), C * k * k)
    b = (0.1 * r.standard_normal(OC)).astype(np.float32)
    dz = r.standard_normal((B, OC, OH, OW)).astype(np.float32)
    hx, hw, hb, hdz = upload(eng, x), upload(eng, w), upload(eng, b), upload(eng, dz)
    hy = eng.lib.CreateBuffer(None, B * OC * OH * OW)
    for act in (0, 1, 2):
        _run_shader(eng, "conv_forward_tiled", [hx, hw, hb], [hy], [*geo, act])
        ref = K.conv_forward_tiled(x, w, b, np.zeros(B * OC * OH * OW), *geo, act)
        assert rel_err(download(eng, hy, (B * OC * OH * OW,)), ref) <= TOL, act
    hdf = eng.lib.CreateBuffer(None, OC * C * k * k)
    sentinel = np.full(OC, 7.0, np.float32)
    hdb = upload(eng, sentinel)
    _run_shader(eng, "conv_backprop_filters_tiled", [hdz, hx], [hdf, hdb], list(geo))
    ref = K.conv_backprop_filters_tiled(dz, x, np.zeros(OC * C * k * k), *geo)
    assert rel_err(download(eng, hdf, (OC * C * k * k,)), ref) <= TOL
    assert np.array_equal(download(eng, hdb, (OC,)), sentinel)
    u = r.standard_normal(x.shape).astype(np.float32)
    hdx = eng.lib.CreateBuffer(None, x.size)
    for act, a in ((0, u), (1, np.maximum(u, 0)), (2, np.tanh(u).astype(np.float32))):
        ha = upload(eng, a)
        _run_shader(eng, "conv_backprop_input_fused", [hdz, hw, ha], [hdx], [*geo, act])
        ref = K.conv_backprop_input_fused(dz, w, a, np.zeros(x.size), *geo, act)
        assert rel_err(download(eng, hdx, (x.size,)), ref) <= TOL, act
        release(eng, ha)
    release(eng, hx, hw, hb, hdz, hy, hdf, hdb, hdx)


def test_tiled_conv_shaders_flat_geometry(eng):
    """Geometry that is not a valid convolution and buffers shorter than the
    geometry take the checked kernels, which follow the shaders' flat index
    arithmetic with reads past a buffer returning 0 and writes dropped."""
    r = rng(4242)
    geo = (2, 2, 5, 4, 3, 2, 5, 3)
    B, C, H, W, OC, ks, OH, OW = geo
    x = r.standard_normal(B * C * H * W - 5).astype(np.float32)
    f = r.standard_normal(OC * C * ks * ks).astype(np.float32)
    bias = r.standard_normal(OC - 1).astype(np.float32)
    out0 = r.standard_normal(B * OC * OH * OW - 4).astype(np.float32)
    hx, hf, hb = upload(eng, x), upload(eng, f), upload(eng, bias)
    for act in (0, 1, 2):
        ho = upload(eng, out0)
        _run_shader(eng, "conv_forward_tiled", [hx, hf, hb], [ho], [*geo, act])
        assert rel_err(download(eng, ho, out0.shape), K.conv_forward_tiled(x, f, bias, out0, *geo, act)) <= 1e-5
        release(eng, ho)
    dz = r.standard_normal(B * OC * OH * OW - 3).astype(np.float32)
    dF0 = r.standard_normal(OC * C * ks * ks - 2).astype(np.float32)
    hdz, hdf = upload(eng, dz), upload(eng, dF0)
    _run_shader(eng, "conv_backprop_filters_tiled", [hdz, hx], [hdf], list(geo))
    assert rel_err(download(eng, hdf, dF0.shape), K.conv_backprop_filters_tiled(dz, x, dF0, *geo)) <= 1e-5
    ap = r.standard_normal(B * C * H * W - 7).astype(np.float32)
    dx0 = r.standard_normal(B * C * H * W - 1).astype(np.float32)
    ha = upload(eng, ap)
    for act in (0, 1, 2):
        hdx = upload(eng, dx0)
        _run_shader(eng, "conv_backprop_input_fused", [hdz, hf, ha], [hdx], [*geo, act])
        ref = K.conv_backprop_input_fused(dz, f, ap, dx0, *geo, act)
        assert rel_err(download(eng, hdx, dx0.shape), ref) <= 1e-5
        release(eng, hdx)
    release(eng, hx, hf, hb, hdz, hdf, ha)
