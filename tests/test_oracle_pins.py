"""CPU pins of the float64 oracle (oracle/kernels.py, oracle/engine64.py).

Every oracle function is checked against something that does not restate its
own formula: torch CPU library routines and autograd (float64), brute-force
scalar loops written from the HLSL text, adjoint identities and central finite
differences (the reference's own protocol, nn_verify.py:63-141).  The golden
end-to-end pin (the reference's logged UNet run) is test_reference_log.py.
"""
import numpy as np
import pytest

from oracle import engine64 as E
from oracle import kernels as K

torch = pytest.importorskip("torch")
F = torch.nn.functional


def t64(a, grad=False):
    return torch.tensor(np.asarray(a, dtype=np.float64), requires_grad=grad)


def close(a, b, tol=1e-10):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    scale = max(1.0, float(np.max(np.abs(b))) if b.size else 1.0)
    assert float(np.max(np.abs(a - b))) <= tol * scale if a.size else True


rng = np.random.default_rng

CONV = [(2, 3, 9, 8, 4, 3, 1, 1), (1, 2, 11, 11, 3, 5, 2, 2), (2, 4, 7, 7, 5, 3, 3, 0), (1, 3, 30, 30, 2, 11, 4, 2),
        (2, 5, 6, 6, 3, 1, 1, 0)]


# --------------------------------------------- direct valid convolutions
TILED = [(2, 3, 9, 8, 4, 3), (1, 5, 7, 7, 6, 1), (3, 2, 12, 10, 5, 5), (2, 4, 6, 6, 3, 6)]


@pytest.mark.parametrize("B,C,H,W,OC,k", TILED)
def test_tiled_convs_valid_geometry_vs_torch(B, C, H, W, OC, k):
    """K.conv_forward_tiled / conv_backprop_filters_tiled /
    conv_backprop_input_fused on valid geometry (stride 1, no padding)
    against torch's conv2d, conv2d_weight and autograd through the previous
    layer's ReLU / tanh (dA = 1 - a² is tanh's derivative at its output)."""
    r = rng(B * 100 + C * 10 + k)
    OH, OW = H - k + 1, W - k + 1
    x, w, b = r.standard_normal((B, C, H, W)), r.standard_normal((OC, C, k, k)), r.standard_normal(OC)
    dz = r.standard_normal((B, OC, OH, OW))
    geo = (B, C, H, W, OC, k, OH, OW)
    z = F.conv2d(t64(x), t64(w), t64(b))
    for act, ref in ((0, z), (1, F.relu(z)), (2, torch.tanh(z)), (7, z)):
        out = K.conv_forward_tiled(x, w, b, np.zeros(B * OC * OH * OW), *geo, act)
        close(out.reshape(z.shape), ref.numpy())
    dF = K.conv_backprop_filters_tiled(dz, x, np.zeros(OC * C * k * k), *geo)
    close(dF.reshape(w.shape), torch.nn.grad.conv2d_weight(t64(x), w.shape, t64(dz)).numpy())
    u = r.standard_normal(x.shape)
    for act, fn in ((0, lambda v: v), (1, F.relu), (2, torch.tanh)):
        ut = t64(u, True)
        a = fn(ut)
        F.conv2d(a, t64(w)).backward(t64(dz))
        dx = K.conv_backprop_input_fused(dz, w, a.detach().numpy(), np.zeros(x.size), *geo, act)
        close(dx.reshape(x.shape), ut.grad.numpy())


def _tiled_brute(kind, bufs, geo, act=0):
    """Scalar loops written from the three HLSL texts, with the D3D11 rule
    for out-of-range reads (0) and writes (dropped); 32-bit index math."""
    B, C, H, W, OC, ks, OH, OW = geo
    M32 = 0xFFFFFFFF

    def rd(a, i):
        i &= M32
        return float(a[i]) if i < len(a) else 0.0

    out = list(bufs[-1])

    def wr(i, v):
        i &= M32
        if i < len(out):
            out[i] = v
    if kind == "fwd":
        x, f, bias = bufs[:3]
        K_ = C * ks * ks
        for row in range(OC):
            for col in range(B * OH * OW):
                b, pix = col // (OH * OW), col % (OH * OW)
                oh, ow = pix // OW, pix % OW
                acc = 0.0
                for t in range(K_):
                    ic, kk = t // (ks * ks), t % (ks * ks)
                    acc += rd(f, row * K_ + t) * rd(x, b * (C * H * W) + ic * (H * W) + (oh + kk // ks) * W
                                                   + ow + kk % ks)
                zz = acc + rd(bias, row)
                a = max(0.0, zz) if act == 1 else (np.tanh(zz) if act == 2 else zz)
                wr(b * (OC * OH * OW) + row * (OH * OW) + pix, a)
    elif kind == "dw":
        dz, x = bufs[:2]
        tr = C * ks * ks
        for row in range(OC):
            for col in range(tr):
                ic, kk = col // (ks * ks), col % (ks * ks)
                acc = 0.0
                for k_idx in range(B * OH * OW):
                    b, p = k_idx // (OH * OW), k_idx % (OH * OW)
                    acc += rd(dz, b * (OC * OH * OW) + row * (OH * OW) + p) * \
                        rd(x, b * (C * H * W) + ic * (H * W) + (p // OW + kk // ks) * W + p % OW + kk % ks)
                wr(row * tr + col, acc)
    else:
        dz, f, ap = bufs[:3]
        for g in range(B * C * H * W):
            iw, ih, ic, b = g % W, (g // W) % H, (g // (W * H)) % C, g // (C * H * W)
            acc = 0.0
            for oc in range(OC):
                for kh in range(ks):
                    oh = ih - kh
                    if 0 <= oh < OH:
                        for kw in range(ks):
                            ow = iw - kw
                            if 0 <= ow < OW:
                                acc += rd(dz, b * (OC * OH * OW) + oc * (OH * OW) + oh * OW + ow) * \
                                    rd(f, oc * (C * ks * ks) + ic * (ks * ks) + kh * ks + kw)
            a = rd(ap, g)
            dA = (1.0 if a > 0 else 0.0) if act == 1 else (1.0 - a * a if act == 2 else 1.0)
            wr(g, acc * dA)
    return np.array(out)


def test_tiled_convs_flat_semantics_brute_force():
    """Geometry that is not a valid convolution (an output taller than the
    input allows, so patch rows run into the next row / plane) and buffers
    shorter than the geometry: the oracle follows the shaders' flat index
    arithmetic and the D3D11 out-of-range rules exactly."""
    r = rng(55)
    geo = (2, 2, 5, 4, 3, 2, 5, 3)          # valid would be OH = 4
    B, C, H, W, OC, ks, OH, OW = geo
    x = r.standard_normal(B * C * H * W - 5)  # short input: the last reads return 0
    f = r.standard_normal(OC * C * ks * ks)
    bias = r.standard_normal(OC - 1)         # short bias
    out0 = r.standard_normal(B * OC * OH * OW - 4)   # short output: writes dropped
    for act in (0, 1, 2):
        close(K.conv_forward_tiled(x, f, bias, out0, *geo, act), _tiled_brute("fwd", [x, f, bias, out0], geo, act))
    dz = r.standard_normal(B * OC * OH * OW - 3)
    dF0 = r.standard_normal(OC * C * ks * ks - 2)
    close(K.conv_backprop_filters_tiled(dz, x, dF0, *geo), _tiled_brute("dw", [dz, x, dF0], geo))
    ap = r.standard_normal(B * C * H * W - 7)
    dx0 = r.standard_normal(B * C * H * W - 1)
    for act in (0, 1, 2):
        close(K.conv_backprop_input_fused(dz, f, ap, dx0, *geo, act),
              _tiled_brute("dx", [dz, f, ap, dx0], geo, act))


# ------------------------------------------------------------------ conv
@pytest.mark.parametrize("B,C,H,W,OC,k,s,p", CONV)
def test_conv_forward_vs_torch(B, C, H, W, OC, k, s, p):
    r = rng(B + C + k + s)
    x, w, b = r.standard_normal((B, C, H, W)), r.standard_normal((OC, C, k, k)), r.standard_normal(OC)
    z = F.conv2d(t64(x), t64(w), t64(b), stride=s, padding=p).numpy()
    close(K.conv_forward(x, w, b, s, p, 0), z)
    close(K.conv_forward(x, w, b, s, p, 1), np.maximum(z, 0))
    close(K.conv_forward(x, w, b, s, p, 2), np.tanh(z))


@pytest.mark.parametrize("B,C,H,W,OC,k,s,p", CONV)
def test_conv_backward_vs_torch_library(B, C, H, W, OC, k, s, p):
    r = rng(7 * (B + C + k + s))
    x, w = r.standard_normal((B, C, H, W)), r.standard_normal((OC, C, k, k))
    OH, OW = K.conv_out_hw(H, W, k, s, p)
    dy = r.standard_normal((B, OC, OH, OW))
    dW, db, dX = K.conv_backward(dy, None, x, w, s, p, 0)
    close(dW, torch.nn.grad.conv2d_weight(t64(x), w.shape, t64(dy), stride=s, padding=p).numpy())
    close(dX, torch.nn.grad.conv2d_input(x.shape, t64(w), t64(dy), stride=s, padding=p).numpy())
    close(db, dy.sum(axis=(0, 2, 3)))


def test_conv_backward_relu_mask_matches_autograd():
    """act == 1: the gradient of relu(conv(x)) (mask from the post-ReLU
    output, nn_conv_grad_reshape_relu.hlsl:36)."""
    r = rng(3)
    x, w, b = r.standard_normal((2, 3, 8, 8)), r.standard_normal((5, 3, 3, 3)), r.standard_normal(5)
    xt, wt, bt = t64(x, True), t64(w, True), t64(b, True)
    y = F.relu(F.conv2d(xt, wt, bt, padding=1))
    dy = r.standard_normal(y.shape)
    y.backward(t64(dy))
    dW, db, dX = K.conv_backward(dy, y.detach().numpy(), x, w, 1, 1, 1)
    close(dW, wt.grad.numpy())
    close(db, bt.grad.numpy())
    close(dX, xt.grad.numpy())


def test_conv_backward_tanh_applies_no_derivative():
    """act == 2 backward uses dy unmasked and without tanh' (engine.cpp:816-835
    only special-cases actType == 1)."""
    r = rng(4)
    x, w = r.standard_normal((1, 2, 6, 6)), r.standard_normal((3, 2, 3, 3))
    dy = r.standard_normal((1, 3, 4, 4))
    y = np.tanh(K.conv_forward(x, w, np.zeros(3), 1, 0, 0))
    for a, c in zip(K.conv_backward(dy, y, x, w, 1, 0, 2), K.conv_backward(dy, None, x, w, 1, 0, 0)):
        close(a, c)


def test_conv_backward_finite_differences():
    """Central differences of L = sum(conv(x, w, b) * dy), eps 1e-6."""
    r = rng(5)
    x, w, b = r.standard_normal((1, 2, 5, 6)), r.standard_normal((3, 2, 3, 3)), r.standard_normal(3)
    dy = r.standard_normal((1, 3, 3, 3))

    def L(x_, w_, b_):
        return float((K.conv_forward(x_, w_, b_, 2, 1, 0) * dy).sum())

    dW, db, dX = K.conv_backward(dy, None, x, w, 2, 1, 0)
    eps = 1e-6
    for arr, grad in ((w, dW), (x, dX), (b, db)):
        num = np.zeros_like(arr)
        for i in range(arr.size):
            a1, a2 = arr.copy(), arr.copy()
            a1.flat[i] += eps
            a2.flat[i] -= eps
            args1 = [a1 if arr is t else t for t in (x, w, b)]
            args2 = [a2 if arr is t else t for t in (x, w, b)]
            num.flat[i] = (L(*args1) - L(*args2)) / (2 * eps)
        close(grad, num, 1e-7)


def test_im2col_col2im_adjoint_and_brute_force():
    r = rng(6)
    B, C, H, W, k, s, p = 2, 3, 7, 6, 3, 2, 1
    x = r.standard_normal((B, C, H, W))
    col = K.im2col(x, k, s, p)
    OH, OW = K.conv_out_hw(H, W, k, s, p)
    # brute force from the shader's index formulas (nn_im2col.hlsl:23-41)
    bf = np.zeros_like(col)
    for row in range(C * k * k):
        ic, kk = divmod(row, k * k)
        kh, kw = divmod(kk, k)
        for c in range(B * OH * OW):
            b, pix = divmod(c, OH * OW)
            oh, ow = divmod(pix, OW)
            ih, iw = oh * s + kh - p, ow * s + kw - p
            if 0 <= ih < H and 0 <= iw < W:
                bf[row, c] = x[b, ic, ih, iw]
    close(col, bf, 0)
    c2 = r.standard_normal(col.shape)
    # <im2col(x), c> == <x, col2im(c)>
    assert abs(float((col * c2).sum()) - float((x * K.col2im(c2, x.shape, k, s, p)).sum())) < 1e-10


@pytest.mark.parametrize("flags", range(4))
def test_flagged_matmul_vs_torch(flags):
    r = rng(flags)
    M, Kd, N = 5, 7, 4
    a = r.standard_normal((M, Kd))
    b = r.standard_normal((Kd, N))
    a_raw = a.T.copy() if flags & 1 else a
    b_raw = b.T.copy() if flags & 2 else b
    close(K.matmul(a_raw.ravel(), b_raw.ravel(), M, Kd, N, flags), torch.matmul(t64(a), t64(b)).numpy())


@pytest.mark.parametrize("tA,tB", [(False, False), (True, False), (False, True), (True, True)])
def test_matmul_backward_vs_autograd(tA, tB):
    """engine64.matmul backward covers the four transpose combinations of
    MatMul.backward (nn_engine.py:913-952)."""
    r = rng(10 + 2 * tA + tB)
    A = r.standard_normal((6, 4) if tA else (4, 6))
    Bm = r.standard_normal((5, 6) if tB else (6, 5))
    At, Bt = t64(A, True), t64(Bm, True)
    out = (At.T if tA else At) @ (Bt.T if tB else Bt)
    g = r.standard_normal(out.shape)
    out.backward(t64(g))
    a, b = E.T(A, True), E.T(Bm, True)
    o = E.matmul(a, b, tA, tB)
    o._backward(g)
    close(a.grad, At.grad.numpy())
    close(b.grad, Bt.grad.numpy())


# --------------------------------------------------------------- maxpool
def _maxpool_brute(x, k, s):
    """Scalar loop of nn_maxpool_forward.hlsl:27-51."""
    B, C, H, W = x.shape
    OH, OW = (H - k) // s + 1, (W - k) // s + 1
    out = np.zeros((B, C, OH, OW))
    idx = np.zeros((B, C, OH, OW), np.uint32)
    for b in range(B):
        for c in range(C):
            for oh in range(OH):
                for ow in range(OW):
                    m, mi = -1e30, 0xFFFFFFFF
                    for ph in range(k):
                        for pw in range(k):
                            ih, iw = oh * s + ph, ow * s + pw
                            if ih < H and iw < W:
                                v = float(x[b, c, ih, iw])
                                if v > m:
                                    m, mi = v, ((b * C + c) * H + ih) * W + iw
                    out[b, c, oh, ow], idx[b, c, oh, ow] = m, mi
    return out, idx


@pytest.mark.parametrize("k,s", [(2, 2), (3, 2), (3, 1), (2, 3)])
def test_maxpool_forward_brute_force_with_ties_and_nan(k, s):
    r = rng(k * 10 + s)
    x = r.integers(-3, 3, (2, 3, 9, 8)).astype(np.float32)   # many ties
    x[0, 0, 0, 0] = np.nan
    x[1, 2, 4, 4] = np.nan
    o, i = K.maxpool_forward(x, k, s)
    bo, bi = _maxpool_brute(x, k, s)
    assert np.array_equal(i, bi)
    close(o, bo, 0)


@pytest.mark.parametrize("k,s", [(2, 2), (3, 2)])
def test_maxpool_vs_torch_tie_free(k, s):
    r = rng(20 + k)
    x = r.permutation(2 * 3 * 13 * 13).reshape(2, 3, 13, 13).astype(np.float64)  # distinct values
    o, i = K.maxpool_forward(x, k, s)
    xt = t64(x, True)
    to, ti = F.max_pool2d(xt, k, s, return_indices=True)
    plane = (np.arange(6).reshape(2, 3, 1, 1) * 13 * 13)
    assert np.array_equal(i.astype(np.int64), ti.numpy() + plane)
    close(o, to.detach().numpy(), 0)
    g = r.standard_normal(o.shape)
    to.backward(t64(g))
    close(K.maxpool_backward(g, i, x.size).reshape(x.shape), xt.grad.numpy())


# ------------------------------------------------------------- batchnorm
def test_batchnorm_vs_torch_training_mode():
    r = rng(30)
    x = r.standard_normal((4, 5, 6, 7)) * 3 + 1
    g, b = r.standard_normal(5), r.standard_normal(5)
    rm, rv = r.standard_normal(5), r.random(5) + 0.5
    xt, gt, bt = t64(x, True), t64(g, True), t64(b, True)
    rmt, rvt = t64(rm), t64(rv)
    y = F.batch_norm(xt, rmt, rvt, gt, bt, training=True, momentum=0.1, eps=1e-5)
    mu, var, nrm, nrv = K.batchnorm_mean_var(x, rm, rv, 0.1, True)
    close(K.batchnorm_forward(x, mu, var, g, b, 1e-5), y.detach().numpy())
    close(nrm, rmt.numpy())
    close(nrv, rvt.numpy())
    dy = r.standard_normal(x.shape)
    y.backward(t64(dy))
    dg, db = K.batchnorm_backward_reduce(x, dy, mu, var, 1e-5)
    close(dg, gt.grad.numpy())
    close(db, bt.grad.numpy())
    close(K.batchnorm_backward_dx(x, dy, mu, var, g, dg, db, 1e-5), xt.grad.numpy(), 1e-9)


# ----------------------------------------------------------- elementwise
def test_activation_grads_vs_autograd():
    r = rng(40)
    x = r.standard_normal(200) * 4
    x[:4] = [0.0, 6.0, -0.0, 3.0]
    g = r.standard_normal(200)
    for fo, fg, tf in [(K.relu, K.relu_grad, F.relu), (K.relu6, K.relu6_grad, lambda v: F.hardtanh(v, 0.0, 6.0)),
                       (lambda v: K.leaky_relu(v, 0.1), lambda gg, v: K.leaky_relu_grad(gg, v, 0.1),
                        lambda v: F.leaky_relu(v, 0.1))]:
        xt = t64(x, True)
        y = tf(xt)
        y.backward(t64(g))
        close(fo(x), y.detach().numpy())
        close(fg(g, x), xt.grad.numpy())
    xt = t64(x, True)
    y = torch.sigmoid(xt)
    y.backward(t64(g))
    close(K.sigmoid(x), y.detach().numpy())
    close(K.sigmoid_grad(g, K.sigmoid(x)), xt.grad.numpy())


def test_bias_ops_vs_autograd():
    r = rng(41)
    A, b, g = r.standard_normal((6, 9)), r.standard_normal(9), r.standard_normal((6, 9))
    At, bt = t64(A, True), t64(b, True)
    y = F.relu(At + bt)
    y.backward(t64(g))
    close(K.bias_relu(A, b), y.detach().numpy())
    a, bb = E.T(A, True), E.T(b, True)
    E.bias_relu(a, bb)._backward(g)
    close(a.grad, At.grad.numpy())
    close(bb.grad, bt.grad.numpy())
    # bias_grad in both layouts it is dispatched with
    close(K.bias_grad(A, 6, 9, 9, 1), A.sum(axis=0))
    close(K.bias_grad(A.T.copy(), 6, 9, 1, 6), A.sum(axis=0))


def test_scale_add_vs_torch_add():
    """K.scale_add (nn_scale_add.hlsl:9) against torch.add(α·a, b, alpha=β), plus
    the identities that a dropped or swapped coefficient breaks."""
    r = rng(43)
    a, b = r.standard_normal(37), r.standard_normal(37)
    for alpha, beta in ((1.5, -0.5), (0.0, 2.0), (-3.0, 0.0), (0.25, 0.75)):
        close(K.scale_add(a, b, alpha, beta), torch.add(t64(a) * alpha, t64(b), alpha=beta).numpy())
    close(K.scale_add(a, b, 1.0, 0.0), a)
    close(K.scale_add(a, b, 0.0, 1.0), b)
    close(K.scale_add(a, a, 2.0, -2.0), np.zeros_like(a))


def test_add_bias_linear_layer_vs_autograd():
    """K.add_bias and the engine's AddBias backward (dA = g, db = column sums
    of g) as the last Linear layer of LeNet / AlexNet uses them: x @ W + b,
    (in, out) weights, against torch autograd."""
    r = rng(43)
    x, W, b = r.standard_normal((5, 7)), r.standard_normal((7, 4)), r.standard_normal(4)
    g = r.standard_normal((5, 4))
    xt, Wt, bt = t64(x, True), t64(W, True), t64(b, True)
    y = xt @ Wt + bt
    y.backward(t64(g))
    close(K.add_bias(x @ W, b), y.detach().numpy())
    xo, Wo, bo = E.T(x, True), E.T(W, True), E.T(b, True)
    out = E.add_bias(E.matmul(xo, Wo), bo)
    close(out.data, y.detach().numpy())
    out._backward(g)
    # the matmul node received dA = g; run it to reach x and W
    mm = out._parents[0]
    mm._backward(mm.grad)
    close(bo.grad, bt.grad.numpy())
    close(Wo.grad, Wt.grad.numpy())
    close(xo.grad, xt.grad.numpy())
    # a bias row broadcast over a single row and over many rows
    close(K.add_bias(np.zeros((1, 4)), b), b[None, :])
    close(K.add_bias(np.ones((300, 4)), b), 1.0 + np.tile(b, (300, 1)))


def test_grad_accum_fan_out_vs_autograd():
    """Gradient accumulation (K.grad_accum, the oracle's only way of adding a
    second gradient to a tensor) through a graph where one tensor feeds three
    consumers, one of them twice, against torch autograd."""
    r = rng(44)
    x = r.standard_normal((3, 6))
    w = r.standard_normal((6, 6))
    xt, wt = t64(x, True), t64(w, True)
    h = xt @ wt
    y = F.relu(h) + torch.sigmoid(h) + h * 1.0 + h
    y.sum().backward()
    xo, wo = E.T(x, True), E.T(w, True)
    ho = E.matmul(xo, wo)
    yo = E.add(E.add(E.add(E.relu(ho), E.sigmoid(ho)), ho), ho)
    yo.backward()
    close(xo.grad, xt.grad.numpy())
    close(wo.grad, wt.grad.numpy())
    # the kernel itself: acc + g, repeated accumulation, float32 operands
    a, g = r.standard_normal(9).astype(np.float32), r.standard_normal(9).astype(np.float32)
    close(K.grad_accum(K.grad_accum(a, g), g), a.astype(np.float64) + 2 * g.astype(np.float64))


def test_pool_resample_plumbing_vs_autograd():
    r = rng(42)
    x = r.standard_normal((2, 3, 4, 5))
    xt = t64(x, True)
    y = F.adaptive_avg_pool2d(xt, 1).reshape(2, 3)
    g = r.standard_normal((2, 3))
    y.backward(t64(g))
    close(K.global_avg_pool(x), y.detach().numpy())
    close(K.global_avg_pool_backward(g, x.shape), xt.grad.numpy())
    for sH, sW in [(2, 2), (3, 2)]:
        xt = t64(x, True)
        y = F.interpolate(xt, scale_factor=(sH, sW), mode="nearest")
        g = r.standard_normal(y.shape)
        y.backward(t64(g))
        close(K.upsample(x, sH, sW), y.detach().numpy())
        close(K.upsample_backward(g, x.shape, sH, sW), xt.grad.numpy())
    a, b = r.standard_normal((2, 3, 4, 4)), r.standard_normal((2, 5, 4, 4))
    close(K.concat([a, b]), torch.cat([t64(a), t64(b)], 1).numpy())
    close(K.slice_channels(K.concat([a, b]), 3, 5), b)


@pytest.mark.parametrize("s,p,k", [(1, 1, 3), (2, 1, 3), (1, 2, 5)])
def test_depthwise_vs_torch_grouped_conv(s, p, k):
    r = rng(50 + s + k)
    x, f, b = r.standard_normal((2, 4, 9, 8)), r.standard_normal((4, 1, k, k)), r.standard_normal(4)
    xt, ft, bt = t64(x, True), t64(f, True), t64(b, True)
    y = F.conv2d(xt, ft, bt, stride=s, padding=p, groups=4)
    close(K.depthwise_forward(x, f, b, s, p), y.detach().numpy())
    dy = r.standard_normal(y.shape)
    y.backward(t64(dy))
    close(K.depthwise_backward_input(dy, f, x.shape, s, p), xt.grad.numpy())
    df, db = K.depthwise_backward_filter(dy, x, k, k, s, p)
    close(df, ft.grad.numpy())
    close(db, bt.grad.numpy())


# ------------------------------------------------------------ losses
def test_softmax_ce_vs_torch():
    r = rng(60)
    z, lab = r.standard_normal((7, 10)) * 3, r.integers(0, 10, 7).astype(np.float32)
    zt = t64(z, True)
    loss = F.cross_entropy(zt, torch.tensor(lab.astype(np.int64)))
    loss.backward()
    close(K.softmax(z), torch.softmax(t64(z), 1).numpy())
    assert abs(K.ce_loss(z, lab) - loss.item()) < 1e-12
    close(K.softmax_ce_grad(K.softmax(z), lab), zt.grad.numpy())


def test_argmax_correct_first_max_wins():
    z = np.array([[1, 3, 3, 0], [2, 2, 2, 2], [0, 0, 5, 5], [1, 0, 0, 0]], np.float32)
    lab = np.array([1, 0, 3, 0], np.float32)
    assert K.argmax_correct(z, lab) == int((np.argmax(z, 1) == lab).sum()) == 3


def test_dice_vs_autograd_mean_loss():
    """Dice grad = d mean_b(1 - 2I/(P+T+1e-6)) / dp (nn_dice_loss_grad.hlsl:22-33)."""
    r = rng(61)
    p, t = r.random((3, 1, 5, 6)), (r.random((3, 1, 5, 6)) < 0.3).astype(np.float64)
    pt = t64(p, True)
    tt = t64(t)
    inter = (pt * tt).sum([1, 2, 3])
    loss = 1 - 2 * inter / (pt.sum([1, 2, 3]) + tt.sum([1, 2, 3]) + 1e-6)
    loss.mean().backward()
    close(K.dice_loss(p, t), loss.detach().numpy())
    close(K.dice_loss_grad(p, t), pt.grad.numpy())


# ------------------------------------------------------------ optimisers
def test_sgd_and_norm_clip_vs_torch():
    r = rng(70)
    ws = [r.standard_normal(n) for n in (5, 17)]
    gs = [r.standard_normal(n) * 3 for n in (5, 17)]
    pts = [t64(w, True) for w in ws]
    for p, g in zip(pts, gs):
        p.grad = t64(g)
    tn = float(torch.nn.utils.clip_grad_norm_(pts, 1.0))
    n, scale = K.grad_norm_scale(gs, 1.0)
    assert abs(n - tn) < 1e-12
    for p, g in zip(pts, gs):
        close(np.asarray(g) * scale, p.grad.numpy())
    # element clip then SGD == torch SGD on clamped gradients
    for w, g in zip(ws, gs):
        pt = t64(w, True)
        pt.grad = torch.clamp(t64(g), -1.0, 1.0)
        torch.optim.SGD([pt], lr=0.05).step()
        close(K.sgd(w, g, 0.05, 1.0), pt.detach().numpy())


@pytest.mark.parametrize("max_norm", [1.0, 1e3], ids=["clipped", "unclipped"])
def test_sgd_clipped_vs_torch(max_norm):
    """SGDBatchClipped's update (K.grad_norm_scale, then K.sgd_clipped per
    tensor) equals torch.optim.SGD stepping on gradients scaled in place by
    clip_grad_norm_ (same coefficient max/(norm + 1e-6))."""
    r = rng(72)
    ws = [r.standard_normal(n) for n in (3, 11, 40)]
    gs = [r.standard_normal(n) * 2 for n in (3, 11, 40)]
    pts = [t64(w, True) for w in ws]
    for p, g in zip(pts, gs):
        p.grad = t64(g)
    torch.nn.utils.clip_grad_norm_(pts, max_norm)
    torch.optim.SGD(pts, lr=0.05).step()
    norm, scale = K.grad_norm_scale(gs, max_norm)
    assert (scale < 1.0) == (max_norm == 1.0)
    for w, g, p in zip(ws, gs, pts):
        close(K.sgd_clipped(w, g, 0.05, scale), p.detach().numpy())


def test_adamw_vs_torch_three_steps():
    """The reference's AdamW (host step size lr*sqrt(1-b2^t)/(1-b1^t), decay
    lr*wd*w on the old weight, element clip) equals torch AdamW on clamped
    gradients with eps_t = eps / sqrt(1 - b2^t)."""
    r = rng(71)
    w0 = r.standard_normal(50)
    lr, b1, b2, eps, wd, clip = 1e-2, 0.9, 0.999, 1e-8, 0.01, 1.0
    pt = t64(w0, True)
    opt = torch.optim.AdamW([pt], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    w, m, v = w0.copy(), np.zeros(50), np.zeros(50)
    for t in (1, 2, 3):
        g = r.standard_normal(50) * 2
        w, m, v = K.adam(w, g, m, v, K.adam_step_size(lr, b1, b2, t), b1, b2, eps, lr * wd, clip)
        pt.grad = torch.clamp(t64(g), -clip, clip)
        opt.param_groups[0]["eps"] = eps / np.sqrt(1 - b2 ** t)
        opt.step()
        close(w, pt.detach().numpy(), 1e-12)


# --------------------------------------------------------- composition
def test_engine64_lenet_vs_autograd():
    """The float64 autograd (topological order, accumulation, fused conv+ReLU,
    max-pool routing, flatten, (in, out) linear weights, bias+ReLU, softmax-CE)
    against torch autograd on the same network."""
    r = rng(80)
    x, lab = r.standard_normal((4, 1, 28, 28)), r.integers(0, 10, 4).astype(np.float32)
    W = {"c1": r.standard_normal((6, 1, 5, 5)) * 0.3, "c1b": r.standard_normal(6) * 0.1,
         "c2": r.standard_normal((16, 6, 5, 5)) * 0.1, "c2b": r.standard_normal(16) * 0.1,
         "l1": r.standard_normal((256, 10)) * 0.1, "l1b": r.standard_normal(10) * 0.1}
    T = {k: t64(v, True) for k, v in W.items()}
    h = F.max_pool2d(F.relu(F.conv2d(t64(x), T["c1"], T["c1b"])), 2)
    h = F.max_pool2d(F.relu(F.conv2d(h, T["c2"], T["c2b"])), 2)
    h = F.relu(h.reshape(4, -1) @ T["l1"] + T["l1b"])
    F.cross_entropy(h, torch.tensor(lab.astype(np.int64))).backward()
    O = {k: E.T(v, True) for k, v in W.items()}
    g = E.maxpool2d(E.conv2d(E.T(x), O["c1"], O["c1b"], 1, 0, 1), 2, 2)
    g = E.maxpool2d(E.conv2d(g, O["c2"], O["c2b"], 1, 0, 1), 2, 2)
    g = E.bias_relu(E.matmul(E.flatten(g), O["l1"]), O["l1b"])
    E.softmax_ce(g, lab).backward()
    for k in W:
        close(O[k].grad, T[k].grad.numpy(), 1e-9)


def test_engine64_mobilenet_block_vs_autograd():
    """BN (training), ReLU6, depthwise, 1x1 convs and a residual add (fan-out
    accumulation) against torch autograd."""
    r = rng(81)
    x = r.standard_normal((2, 8, 6, 6))
    W = {"e": r.standard_normal((24, 8, 1, 1)) * 0.3, "eb": np.zeros(24), "g1": r.random(24) + 0.5,
         "b1": r.standard_normal(24) * 0.1, "d": r.standard_normal((24, 1, 3, 3)) * 0.3, "db": np.zeros(24),
         "g2": r.random(24) + 0.5, "b2": r.standard_normal(24) * 0.1, "p": r.standard_normal((8, 24, 1, 1)) * 0.3,
         "pb": np.zeros(8), "g3": r.random(8) + 0.5, "b3": r.standard_normal(8) * 0.1}
    T = {k: t64(v, True) for k, v in W.items()}
    xt = t64(x, True)

    def bn_t(h, g, b):
        return F.batch_norm(h, None, None, g, b, training=True, eps=1e-5)

    h = F.hardtanh(bn_t(F.conv2d(xt, T["e"], T["eb"]), T["g1"], T["b1"]), 0, 6)
    h = F.hardtanh(bn_t(F.conv2d(h, T["d"], T["db"], padding=1, groups=24), T["g2"], T["b2"]), 0, 6)
    h = bn_t(F.conv2d(h, T["p"], T["pb"]), T["g3"], T["b3"]) + xt
    dy = r.standard_normal(h.shape)
    h.backward(t64(dy))
    O = {k: E.T(v, True) for k, v in W.items()}
    xo = E.T(x, True)
    g = E.relu6(E.batchnorm2d(E.conv2d(xo, O["e"], O["eb"]), O["g1"], O["b1"])[0])
    g = E.relu6(E.batchnorm2d(E.depthwise_conv2d(g, O["d"], O["db"], 1, 1), O["g2"], O["b2"])[0])
    out = E.add(E.batchnorm2d(E.conv2d(g, O["p"], O["pb"]), O["g3"], O["b3"])[0], xo)
    out.grad = dy
    # run the traversal from `out` with the given upstream gradient
    topo, seen, stack = [], set(), [(out, False)]
    while stack:
        v, done = stack.pop()
        if done:
            topo.append(v)
            continue
        if id(v) in seen:
            continue
        seen.add(id(v))
        stack.append((v, True))
        stack.extend((p, False) for p in v._parents if p.requires_grad and id(p) not in seen)
    for v in reversed(topo):
        if v._backward is not None and v.grad is not None:
            v._backward(v.grad)
    close(xo.grad, xt.grad.numpy(), 1e-9)
    for k in ("e", "g1", "b1", "d", "g2", "b2", "p", "g3", "b3"):
        close(O[k].grad, T[k].grad.numpy(), 1e-9)


# ------------------------------------------------------- benchmark steps
def _bn_train(h, g, b):
    return F.batch_norm(h, None, None, g, b, training=True, eps=1e-5)


def test_mobilenet_stack_step_vs_autograd():
    """oracle.models.mobilenet_stack_step (the CPU baseline of the MobileNetV2
    stack) against the same network in torch autograd, then SGD."""
    from oracle import models as OM
    r = rng(90)
    P = OM.mobilenet_stack_params(r)
    for k in P:                                   # non-trivial BN affine terms
        if k.endswith(".g"):
            P[k] = (1 + 0.2 * r.standard_normal(P[k].shape)).astype(np.float32)
        elif k.endswith(".be") or k.endswith(".b"):
            P[k] = (0.1 * r.standard_normal(P[k].shape)).astype(np.float32)
    x = r.standard_normal((2, 16, 12, 12)).astype(np.float32)
    lab = r.integers(0, 10, 2).astype(np.float32)
    T = {k: t64(v, True) for k, v in P.items()}
    h = t64(x)
    for i, (ci, co, s) in enumerate(OM.MBV2_BLOCKS):
        t = F.hardtanh(_bn_train(F.conv2d(h, T[f"b{i}.exp.w"], T[f"b{i}.exp.b"]), T[f"b{i}.bn1.g"],
                                 T[f"b{i}.bn1.be"]), 0, 6)
        t = F.conv2d(t, T[f"b{i}.dw.w"], T[f"b{i}.dw.b"], stride=s, padding=1, groups=ci * 6)
        t = F.hardtanh(_bn_train(t, T[f"b{i}.bn2.g"], T[f"b{i}.bn2.be"]), 0, 6)
        t = _bn_train(F.conv2d(t, T[f"b{i}.proj.w"], T[f"b{i}.proj.b"]), T[f"b{i}.bn3.g"], T[f"b{i}.bn3.be"])
        h = t + h if (s == 1 and ci == co) else t
    z = h.mean(dim=(2, 3)) @ T["fc.w"] + T["fc.b"]
    loss_t = F.cross_entropy(z, torch.tensor(lab.astype(np.int64)))
    loss_t.backward()
    loss, g, new = OM.mobilenet_stack_step(P, x, lab, lr=0.01)
    assert abs(loss - float(loss_t.detach())) < 1e-9
    for k in P:
        close(g[k], T[k].grad.numpy(), 1e-8)
        close(new[k], P[k].astype(np.float64) - 0.01 * T[k].grad.numpy(), 1e-9)


def test_unet_step_vs_autograd():
    """oracle.models.unet_step (the CPU baseline of the UNet configuration) at
    two levels against torch autograd: Dice on the sigmoid output, global-norm
    clip (torch clip_grad_norm_), first Adam step (torch Adam with
    eps_t = eps / sqrt(1 - b2))."""
    from oracle import models as OM
    r = rng(91)
    P = OM.unet_params(r, base=4, levels=2)
    x = r.random((2, 3, 8, 8)).astype(np.float32)
    tg = (r.random((2, 1, 8, 8)) < 0.3).astype(np.float32)
    T = {k: t64(v, True) for k, v in P.items()}

    def cbr(h, n):
        return F.relu(_bn_train(F.conv2d(h, T[n + ".w"], T[n + ".b"], padding=1), T[n + ".g"], T[n + ".be"]))
    h, skips = t64(x), []
    for i in range(2):
        h = cbr(cbr(h, f"e{i}a"), f"e{i}b")
        skips.append(h)
        h = F.max_pool2d(h, 2)
    h = cbr(cbr(h, "ba"), "bb")
    for i in reversed(range(2)):
        h = torch.cat([F.interpolate(h, scale_factor=2, mode="nearest"), skips[i]], dim=1)
        h = cbr(cbr(h, f"d{i}a"), f"d{i}b")
    p = torch.sigmoid(F.conv2d(h, T["head.w"], T["head.b"]))
    tt = t64(tg)
    inter = (p * tt).sum([1, 2, 3])
    dl = 1 - 2 * inter / (p.sum([1, 2, 3]) + tt.sum([1, 2, 3]) + 1e-6)
    dl.mean().backward()
    loss, g, new = OM.unet_step(P, x, tg, levels=2, lr=1e-3, max_norm=0.05)
    assert abs(loss - float(dl.mean())) < 1e-12
    for k in P:
        close(g[k], T[k].grad.numpy(), 1e-8)
    params = [T[k] for k in sorted(P)]
    torch.nn.utils.clip_grad_norm_(params, 0.05)
    opt = torch.optim.Adam(params, lr=1e-3, eps=1e-8 / np.sqrt(1 - 0.999))
    opt.step()
    for k in P:
        close(new[k], T[k].detach().numpy(), 1e-9)
