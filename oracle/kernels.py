"""NumPy float64 restatement of the reference kernels on the backward path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / the timed CPU baseline.

Every function restates the arithmetic of one HLSL kernel (or one C++
composition in ``engine.cpp``) of raviadi12/directcompute_torch, in float64,
from the shader source text.  Citations are ``file:line`` relative to the
reference tree.  Layout conventions are the reference's: NCHW activations,
``[OC, C, kH, kW]`` filters, ``(in, out)`` linear weights, row-major GEMMs.

Reduction order: the reference reduces with 256 thread-strided partials and a
shared-memory tree.  In float64 the summation order changes results by far
less than the 1e-4 parity tolerance, so plain ``np.sum`` / BLAS is used; the
order is *not* part of the parity contract.

Pinning status of each function is recorded in ``tests/test_oracle_pins.py``
(closed forms, brute-force loops, ``torch`` CPU library routines, finite
differences).
"""
from __future__ import annotations

import numpy as np

F64 = np.float64
IDX_NONE = np.uint32(0xFFFFFFFF)


def _f64(a):
    return np.asarray(a, dtype=F64)


# ----------------------------------------------------------------------------
# Convolution: im2col / col2im / fused forward / fused backward
# ----------------------------------------------------------------------------

def conv_out_hw(H, W, k, s, p):
    """Output geometry, floor mode (engine.cpp:758-761)."""
    return (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1


def im2col(x, k, s, p):
    """col[(c,kh,kw), (b,oh,ow)] = x[b,c,oh*s+kh-p,ow*s+kw-p] or 0.

    Restates nn_im2col.hlsl:23-41 (row = c*k*k + kh*k + kw,
    column = b*OH*OW + oh*OW + ow, zero padding).
    """
    x = _f64(x)
    B, C, H, W = x.shape
    OH, OW = conv_out_hw(H, W, k, s, p)
    xp = np.zeros((B, C, H + 2 * p + k, W + 2 * p + k), dtype=F64)
    xp[:, :, p:p + H, p:p + W] = x
    col = np.empty((C, k, k, B, OH, OW), dtype=F64)
    for kh in range(k):
        for kw in range(k):
            sl = xp[:, :, kh:kh + s * OH:s, kw:kw + s * OW:s][:, :, :OH, :OW]
            col[:, kh, kw] = sl.transpose(1, 0, 2, 3)
    return col.reshape(C * k * k, B * OH * OW)


def col2im(dcol, x_shape, k, s, p):
    """Inverse gather of im2col: dx[b,c,ih,iw] = sum over (kh,kw) with
    (ih+p-kh) divisible by s and in range (nn_col2im.hlsl:21-45).

    Implemented as the adjoint scatter-add of :func:`im2col`, which is the same
    sum (every (kh,kw,oh,ow) with oh*s+kh-p == ih contributes once).
    """
    B, C, H, W = x_shape
    OH, OW = conv_out_hw(H, W, k, s, p)
    d = _f64(dcol).reshape(C, k, k, B, OH, OW)
    xp = np.zeros((B, C, H + 2 * p + k, W + 2 * p + k), dtype=F64)
    for kh in range(k):
        for kw in range(k):
            xp[:, :, kh:kh + s * OH:s, kw:kw + s * OW:s][:, :, :OH, :OW] += d[:, kh, kw].transpose(1, 0, 2, 3)
    return xp[:, :, p:p + H, p:p + W].copy()


def conv_forward(x, Wt, b, s, p, act):
    """ConvForwardFused (engine.cpp:751-798): im2col, GEMM W·col, then
    conv_reshape (nn_conv_reshape.hlsl:19-29): + bias, act 0 = identity,
    1 = ReLU (max(0,z)), 2 = tanh; output NCHW."""
    x = _f64(x)
    Wt = _f64(Wt)
    B, C, H, W = x.shape
    OC, _, k, _ = Wt.shape
    OH, OW = conv_out_hw(H, W, k, s, p)
    col = im2col(x, k, s, p)
    z = Wt.reshape(OC, -1) @ col + _f64(b).reshape(OC, 1)
    if act == 1:
        z = np.maximum(z, 0.0)
    elif act == 2:
        z = np.tanh(z)
    return z.reshape(OC, B, OH, OW).transpose(1, 0, 2, 3).copy()


def conv_grad_reshape(dy, y=None, act=0):
    """G[oc, b*OH*OW + pix] from NCHW dy; with act==1 and a forward output y the
    ReLU mask zeroes entries where y <= 0 (nn_conv_grad_reshape_relu.hlsl:33-38,
    nn_conv_grad_reshape.hlsl:21-27).  NaN in y keeps the gradient, as
    ``y <= 0`` is false for NaN."""
    dy = _f64(dy)
    if act == 1 and y is not None:
        y = np.asarray(y)
        dy = np.where(y <= 0, 0.0, dy)
    B, OC, OH, OW = dy.shape
    return dy.transpose(1, 0, 2, 3).reshape(OC, B * OH * OW)


def conv_backward(dy, y, x, Wt, s, p, act, need_x=True, need_w=True, need_b=True):
    """ConvBackwardFused (engine.cpp:802-878).

    G = conv_grad_reshape(_relu)(dy, y) (ReLU mask only for act==1; act==2
    applies no derivative -- kept as the reference behaves);
    dW = G · colᵀ (MatMulDispatch flags=2, engine.cpp:838-842);
    db = row sums of G (bias_grad, engine.cpp:844-855);
    dX = col2im(Wᵀ · G) (flags=1 GEMM + col2im, engine.cpp:857-873).
    Returns (dW, db, dX) with None for gradients not requested.
    """
    x = _f64(x)
    Wt = _f64(Wt)
    B, C, H, W = x.shape
    OC, _, k, _ = Wt.shape
    G = conv_grad_reshape(dy, y, act)
    dW = db = dX = None
    if need_w:
        col = im2col(x, k, s, p)
        dW = (G @ col.T).reshape(Wt.shape)
    if need_b:
        db = G.sum(axis=1)
    if need_x:
        dcol = Wt.reshape(OC, -1).T @ G
        dX = col2im(dcol, x.shape, k, s, p)
    return dW, db, dX


# The three direct valid convolutions the reference compiles (nn_engine.py:148):
# stride 1, no padding, square kernel ks, constants {batch, inC, inH, inW, outC,
# ks, outH, outW, act}.  They work on flat buffers, with the shaders' own 32-bit
# index arithmetic (wrapping) and the D3D11 rule that a read past a buffer
# returns 0 and a write past it is dropped, so any geometry is defined; with
# outH = inH - ks + 1 and outW = inW - ks + 1 they are ordinary valid
# convolutions.  Each returns the updated output buffer.

def _u32(a):
    return np.asarray(a, dtype=np.int64) & 0xFFFFFFFF


def _rd(buf, idx):
    """buf[idx] with reads past the buffer returning 0."""
    buf = _f64(buf).reshape(-1)
    idx = _u32(idx)
    ok = idx < buf.size
    return np.where(ok, buf[np.where(ok, idx, 0)], 0.0)


def _wr(out, idx, vals):
    """out[idx] = vals, dropping writes past the buffer."""
    out = _f64(out).reshape(-1).copy()
    idx = _u32(idx)
    vals = np.broadcast_to(_f64(vals), idx.shape).reshape(-1)
    idx = idx.reshape(-1)
    ok = idx < out.size
    out[idx[ok]] = vals[ok]
    return out


def conv_forward_tiled(x, F, bias, out, batch, inC, inH, inW, outC, ks, outH, outW, act):
    """nn_conv_forward_tiled.hlsl:22-71.  M = outC rows of filters (row-major,
    K = inC*ks*ks), N = batch*outH*outW columns; the input patch of column
    (b, oh, ow) at k = (ic, kh, kw) is input[b*inC*inH*inW + ic*inH*inW +
    (oh+kh)*inW + ow+kw]; z = acc + bias[row]; act 1 = max(0, z), 2 = tanh,
    else z; written at output[b*outC*outH*outW + row*outH*outW + pixel]."""
    M, N, K, P = outC, batch * outH * outW, inC * ks * ks, outH * outW
    col = np.arange(N, dtype=np.int64)
    b, pix = col // P, col % P
    oh, ow = pix // outW, pix % outW
    t = np.arange(K, dtype=np.int64)
    ic, kk = t // (ks * ks), t % (ks * ks)
    kh, kw = kk // ks, kk % ks
    xi = (b[None, :] * (inC * inH * inW) + ic[:, None] * (inH * inW)
          + (oh[None, :] + kh[:, None]) * inW + (ow[None, :] + kw[:, None]))
    patches = _rd(x, xi)                                         # K x N
    rows = np.arange(M, dtype=np.int64)
    Fm = _rd(F, rows[:, None] * K + t[None, :])                  # M x K
    z = Fm @ patches + _rd(bias, rows)[:, None]
    if act == 1:
        z = np.maximum(0.0, z)
    elif act == 2:
        z = np.tanh(z)
    oi = b[None, :] * (outC * P) + rows[:, None] * P + pix[None, :]
    return _wr(out, oi, z)


def conv_backprop_filters_tiled(dZ, x, dF, batch, inC, inH, inW, outC, ks, outH, outW):
    """nn_conv_backprop_filters_tiled.hlsl:21-74.  dF[row*tr + col] (tr =
    inC*ks*ks, col = (ic, kh, kw)) = Σ over k in batch*outH*outW of
    dZ[b*outC*outH*outW + row*outH*outW + p] * input[b*inC*inH*inW +
    ic*inH*inW + (oh+kh)*inW + ow+kw].  No activation mask; the dB buffer
    the dispatch binds is never written."""
    M, N, tr, P = outC, batch * outH * outW, inC * ks * ks, outH * outW
    k = np.arange(N, dtype=np.int64)
    b, p = k // P, k % P
    oh, ow = p // outW, p % outW
    rows = np.arange(M, dtype=np.int64)
    dz = _rd(dZ, b[None, :] * (outC * P) + rows[:, None] * P + p[None, :])     # M x N
    c = np.arange(tr, dtype=np.int64)
    ic, kk = c // (ks * ks), c % (ks * ks)
    kh, kw = kk // ks, kk % ks
    xi = (b[:, None] * (inC * inH * inW) + ic[None, :] * (inH * inW)
          + (oh[:, None] + kh[None, :]) * inW + (ow[:, None] + kw[None, :]))
    return _wr(dF, rows[:, None] * tr + c[None, :], dz @ _rd(x, xi))


def conv_backprop_input_fused(dZ, F, a_prev, dx, batch, inC, inH, inW, outC, ks, outH, outW,
                              prev_act):
    """nn_conv_backprop_input_fused.hlsl:19-50.  For each input element gid <
    batch*inC*inH*inW: acc = Σ_{oc, kh, kw} dZ[b, oc, ih-kh, iw-kw] *
    filters[oc, ic, kh, kw] over the in-range (oh, ow); dA from a =
    A_prev[gid]: prevActType 1 -> (a > 0 ? 1 : 0), 2 -> 1 - a², else 1;
    dInput[gid] = acc * dA."""
    total = batch * inC * inH * inW
    g = np.arange(total, dtype=np.int64)
    iw, ih = g % inW, (g // inW) % inH
    ic, b = (g // (inW * inH)) % inC, g // (inC * inH * inW)
    acc = np.zeros(total)
    for oc in range(outC):
        for kh in range(ks):
            oh = ih - kh
            for kw in range(ks):
                ow = iw - kw
                ok = (oh >= 0) & (oh < outH) & (ow >= 0) & (ow < outW)
                zi = b * (outC * outH * outW) + oc * (outH * outW) + np.where(ok, oh * outW + ow, 0)
                fv = _rd(F, np.full(1, oc * (inC * ks * ks) + kh * ks + kw) + ic * (ks * ks))
                acc += np.where(ok, _rd(dZ, zi) * fv, 0.0)
    a = _rd(a_prev, g)
    if prev_act == 1:
        dA = np.where(a > 0.0, 1.0, 0.0)
    elif prev_act == 2:
        dA = 1.0 - a * a
    else:
        dA = np.ones_like(a)
    return _wr(dx, g, acc * dA)


def matmul(A, Bm, M, K, N, flags):
    """Flagged GEMM shared by matmul_{heavy,dgpu,universal,reduce}: bit0 means A
    is stored K×M (A[k*M+m]), bit1 means B is stored N×K (B[n*K+k]); C is M×N
    row-major (nn_matmul_heavy.hlsl:44-47, nn_matmul_reduce.hlsl:38-41)."""
    A = _f64(A).reshape(-1)
    Bm = _f64(Bm).reshape(-1)
    a = A[:M * K].reshape(K, M).T if flags & 1 else A[:M * K].reshape(M, K)
    b = Bm[:K * N].reshape(N, K).T if flags & 2 else Bm[:K * N].reshape(K, N)
    return a @ b


# ----------------------------------------------------------------------------
# Max pooling
# ----------------------------------------------------------------------------

def maxpool_forward(x, k, s):
    """Window scan of nn_maxpool_forward.hlsl:27-51: no padding, floor mode,
    scan ph outer / pw inner, strict ``>``, init -1e30 and index 0xFFFFFFFF;
    the index is the absolute flat NCHW input index.  Vectorised over all
    windows but with the same scan order and comparison, so NaN is never
    selected and ties keep the first candidate.  Returns (out float64,
    idx uint32)."""
    x = np.asarray(x)
    B, C, H, W = x.shape
    OH, OW = (H - k) // s + 1, (W - k) // s + 1
    xv = x.astype(F64)
    best = np.full((B, C, OH, OW), -1e30, dtype=F64)
    bidx = np.full((B, C, OH, OW), IDX_NONE, dtype=np.uint32)
    base = (np.arange(B * C, dtype=np.int64) * H * W).reshape(B, C, 1, 1)
    oh = np.arange(OH).reshape(1, 1, OH, 1)
    ow = np.arange(OW).reshape(1, 1, 1, OW)
    for ph in range(k):
        for pw in range(k):
            ih = oh * s + ph
            iw = ow * s + pw
            ok = (ih < H) & (iw < W)
            ihc = np.minimum(ih, H - 1)
            iwc = np.minimum(iw, W - 1)
            val = xv[:, :, ihc[0, 0, :, 0], :][:, :, :, iwc[0, 0, 0, :]]
            take = ok & (val > best)
            best = np.where(take, val, best)
            flat = (base + ihc * W + iwc).astype(np.uint32)
            bidx = np.where(take, flat, bidx)
    return best, bidx


def maxpool_backward(dz, idx, x_size):
    """Argmax routing of nn_maxpool_backward.hlsl:21-24 after the zero clear of
    MaxPoolBackwardFused (engine.cpp:916-918).  The reference *stores*
    dX[idx]=dZ, which races when windows overlap; this restatement sums the
    contributions (np.add.at), the deterministic semantics the HIP kernel
    implements.  For disjoint windows store and sum coincide exactly."""
    out = np.zeros(x_size, dtype=F64)
    idx = np.asarray(idx).reshape(-1).astype(np.int64)
    dz = _f64(dz).reshape(-1)
    keep = idx != int(IDX_NONE)
    np.add.at(out, idx[keep], dz[keep])
    return out


# ----------------------------------------------------------------------------
# Batch normalisation (training mode)
# ----------------------------------------------------------------------------

def batchnorm_mean_var(x, running_mean=None, running_var=None, momentum=0.1, training=True):
    """nn_batchnorm_mean_var.hlsl:27-59: one-pass moments, var = max(0,
    E[x²]-E[x]²); running stats use the unbiased var·m/max(1,m-1).
    Returns (mean, var, new_running_mean, new_running_var)."""
    x = _f64(x)
    B, C, H, W = x.shape
    m = B * H * W
    s1 = x.sum(axis=(0, 2, 3))
    s2 = (x * x).sum(axis=(0, 2, 3))
    mean = s1 / m
    var = np.maximum(0.0, s2 / m - mean * mean)
    rm = rv = None
    if running_mean is not None and training:
        unb = var * (m / max(1.0, m - 1.0))
        rm = (1.0 - momentum) * _f64(running_mean) + momentum * mean
        rv = (1.0 - momentum) * _f64(running_var) + momentum * unb
    return mean, var, rm, rv


def batchnorm_forward(x, mean, var, gamma, beta, eps):
    """nn_batchnorm_forward.hlsl:24-34: (x-μ)·(1/√(σ²+ε))·γ+β."""
    x = _f64(x)
    sh = (1, -1, 1, 1)
    rstd = 1.0 / np.sqrt(_f64(var) + eps)
    return (x - _f64(mean).reshape(sh)) * rstd.reshape(sh) * _f64(gamma).reshape(sh) + _f64(beta).reshape(sh)


def batchnorm_backward_reduce(x, dy, mean, var, eps):
    """nn_batchnorm_backward_reduce.hlsl:27-60: dγ = Σ dy·x̂, dβ = Σ dy."""
    x = _f64(x)
    dy = _f64(dy)
    sh = (1, -1, 1, 1)
    rstd = 1.0 / np.sqrt(_f64(var) + eps)
    xhat = (x - _f64(mean).reshape(sh)) * rstd.reshape(sh)
    return (dy * xhat).sum(axis=(0, 2, 3)), dy.sum(axis=(0, 2, 3))


def batchnorm_backward_dx(x, dy, mean, var, gamma, dgamma, dbeta, eps):
    """nn_batchnorm_backward_dx.hlsl:26-38:
    dx = γ·rstd·(dy − (dβ + x̂·dγ)/(N·S))."""
    x = _f64(x)
    dy = _f64(dy)
    B, C, H, W = x.shape
    sh = (1, -1, 1, 1)
    rstd = (1.0 / np.sqrt(_f64(var) + eps)).reshape(sh)
    xhat = (x - _f64(mean).reshape(sh)) * rstd
    m = float(B * H * W)
    return (_f64(gamma).reshape(sh) * rstd) * (dy - (_f64(dbeta).reshape(sh) + xhat * _f64(dgamma).reshape(sh)) / m)


# ----------------------------------------------------------------------------
# Elementwise activations and their gradients
# ----------------------------------------------------------------------------

def relu(x):
    """nn_relu.hlsl:4-5."""
    return np.maximum(_f64(x), 0.0)


def relu_grad(g, inp):
    """nn_relu_grad.hlsl:7-9: inp > 0 ? g : 0 (NaN inp -> 0)."""
    return np.where(_f64(inp) > 0, _f64(g), 0.0)


def relu6(x):
    """nn_relu6.hlsl:7-10."""
    return np.minimum(np.maximum(_f64(x), 0.0), 6.0)


def relu6_grad(g, x):
    """nn_relu6_grad.hlsl:8-11: (0 < x < 6) ? g : 0."""
    x = _f64(x)
    return np.where((x > 0.0) & (x < 6.0), _f64(g), 0.0)


def sigmoid(x):
    """nn_sigmoid.hlsl:11-13."""
    return 1.0 / (1.0 + np.exp(-_f64(x)))


def sigmoid_grad(dy, y):
    """nn_sigmoid_grad.hlsl:11-14: dy·y·(1−y), y the forward output."""
    y = _f64(y)
    return _f64(dy) * y * (1.0 - y)


def leaky_relu(x, alpha):
    """nn_leaky_relu.hlsl:11-15."""
    x = _f64(x)
    return np.where(x > 0.0, x, x * alpha)


def leaky_relu_grad(dy, x, alpha):
    """nn_leaky_relu_grad.hlsl:11-16: dy·(x > 0 ? 1 : α)."""
    return _f64(dy) * np.where(_f64(x) > 0.0, 1.0, alpha)


def grad_accum(acc, g):
    """nn_grad_accum.hlsl:6-8: acc += g."""
    return _f64(acc) + _f64(g)


def add(a, b):
    """nn_add.hlsl:6-7."""
    return _f64(a) + _f64(b)


def add_bias(A, b):
    """nn_add_bias.hlsl:6-9: C[i] = A[i] + b[i % N] for A of shape (M, N)."""
    return _f64(A) + _f64(b).reshape(1, -1)


def bias_relu(A, b):
    """nn_bias_relu.hlsl:9-12."""
    return np.maximum(_f64(A) + _f64(b).reshape(1, -1), 0.0)


def bias_grad(G, rows, classes, stride_i, stride_id):
    """nn_bias_grad.hlsl:12-29: g[c] = Σ_i G[i*stride_i + c*stride_id]."""
    G = _f64(G).reshape(-1)
    i = np.arange(rows).reshape(-1, 1)
    c = np.arange(classes).reshape(1, -1)
    idx = i * stride_i + c * stride_id
    ok = idx < G.size
    return np.where(ok, G[np.minimum(idx, G.size - 1)], 0.0).sum(axis=0)


def scale_add(a, b, alpha, beta):
    """nn_scale_add.hlsl: alpha·a + beta·b."""
    return alpha * _f64(a) + beta * _f64(b)


# ----------------------------------------------------------------------------
# Pooling / resampling / channel plumbing
# ----------------------------------------------------------------------------

def global_avg_pool(x):
    """nn_global_avg_pool.hlsl:26-43: mean over H·W per (n,c)."""
    x = _f64(x)
    return x.reshape(x.shape[0], x.shape[1], -1).mean(axis=2)


def global_avg_pool_backward(g, x_shape):
    """nn_global_avg_pool_backward.hlsl:16-19: dx[i] = g[i/S]/S."""
    B, C, H, W = x_shape
    S = H * W
    return np.broadcast_to((_f64(g).reshape(B, C, 1, 1) / S), (B, C, H, W)).copy()


def upsample(x, sH, sW):
    """nn_upsample.hlsl:17-33: nearest, out[h,w] = in[h/sH, w/sW]."""
    return np.repeat(np.repeat(_f64(x), sH, axis=2), sW, axis=3)


def upsample_backward(dy, x_shape, sH, sW):
    """nn_upsample_backward.hlsl:17-44: dX = block sum of dY, bounded by the
    output extent."""
    B, C, H, W = x_shape
    dy = _f64(dy)
    OH, OW = dy.shape[2], dy.shape[3]
    out = np.zeros((B, C, H, W), dtype=F64)
    for sh in range(sH):
        for sw in range(sW):
            hs = np.arange(H) * sH + sh
            ws = np.arange(W) * sW + sw
            hi = np.nonzero(hs < OH)[0]
            wi = np.nonzero(ws < OW)[0]
            out[:, :, hi[:, None], wi[None, :]] += dy[:, :, hs[hi][:, None], ws[wi][None, :]]
    return out


def concat(tensors):
    """Concat forward via concat_insert (nn_concat_insert.hlsl:17-33)."""
    return np.concatenate([_f64(t) for t in tensors], axis=1)


def slice_channels(dy, c_off, c_in):
    """nn_slice.hlsl:17-26: copy channels [c_off, c_off+c_in) of dY."""
    return _f64(dy)[:, c_off:c_off + c_in].copy()


# ----------------------------------------------------------------------------
# Depthwise convolution
# ----------------------------------------------------------------------------

def depthwise_forward(x, f, b, s, p):
    """nn_depthwise_conv_forward.hlsl:24-50."""
    x = _f64(x)
    f = _f64(f)
    B, C, H, W = x.shape
    kH, kW = f.shape[2], f.shape[3]
    OH = (H + 2 * p - kH) // s + 1
    OW = (W + 2 * p - kW) // s + 1
    xp = np.zeros((B, C, H + 2 * p + kH, W + 2 * p + kW), dtype=F64)
    xp[:, :, p:p + H, p:p + W] = x
    out = np.zeros((B, C, OH, OW), dtype=F64)
    for fh in range(kH):
        for fw in range(kW):
            out += xp[:, :, fh:fh + s * OH:s, fw:fw + s * OW:s][:, :, :OH, :OW] * f[:, 0, fh, fw].reshape(1, C, 1, 1)
    return out + _f64(b).reshape(1, C, 1, 1)


def depthwise_backward_input(dy, f, x_shape, s, p):
    """nn_depthwise_conv_backward_input.hlsl:26-51 (gather form; computed here
    as the adjoint scatter, the same sum)."""
    dy = _f64(dy)
    f = _f64(f)
    B, C, H, W = x_shape
    kH, kW = f.shape[2], f.shape[3]
    OH, OW = dy.shape[2], dy.shape[3]
    xp = np.zeros((B, C, H + 2 * p + kH, W + 2 * p + kW), dtype=F64)
    for fh in range(kH):
        for fw in range(kW):
            xp[:, :, fh:fh + s * OH:s, fw:fw + s * OW:s][:, :, :OH, :OW] += dy * f[:, 0, fh, fw].reshape(1, C, 1, 1)
    return xp[:, :, p:p + H, p:p + W].copy()


def depthwise_backward_filter(dy, x, kH, kW, s, p):
    """nn_depthwise_conv_backward_filter.hlsl:30-75: db[c] = Σ dy, and
    df[c,fh,fw] = Σ dy·x_shifted (zero outside).  Returns (df (C,1,kH,kW), db)."""
    dy = _f64(dy)
    x = _f64(x)
    B, C, H, W = x.shape
    OH, OW = dy.shape[2], dy.shape[3]
    xp = np.zeros((B, C, H + 2 * p + kH, W + 2 * p + kW), dtype=F64)
    xp[:, :, p:p + H, p:p + W] = x
    df = np.zeros((C, 1, kH, kW), dtype=F64)
    for fh in range(kH):
        for fw in range(kW):
            df[:, 0, fh, fw] = (dy * xp[:, :, fh:fh + s * OH:s, fw:fw + s * OW:s][:, :, :OH, :OW]).sum(axis=(0, 2, 3))
    return df, dy.sum(axis=(0, 2, 3))


# ----------------------------------------------------------------------------
# Losses and metrics
# ----------------------------------------------------------------------------

def softmax(x):
    """nn_softmax.hlsl:7-11 (max-subtracted exp / sum)."""
    x = _f64(x)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def ce_loss(logits, labels):
    """nn_loss.hlsl:14-43: mean over the batch of −(z[label] − max − log Σexp);
    labels are float values truncated to uint."""
    z = _f64(logits)
    lab = np.asarray(labels).reshape(-1).astype(np.float32).astype(np.int64)
    mx = z.max(axis=1)
    lse = np.log(np.exp(z - mx[:, None]).sum(axis=1))
    return float(np.mean(-(z[np.arange(z.shape[0]), lab] - mx - lse)))


def softmax_ce_grad(p, labels):
    """nn_softmax_ce_grad.hlsl:8-11: (softmax − onehot)/B, where the one-hot
    test is ``labels[b] == (float)j``."""
    p = _f64(p)
    B, K = p.shape
    lab = np.asarray(labels, dtype=np.float32).reshape(-1)
    onehot = (lab[:, None] == np.arange(K, dtype=np.float32)[None, :]).astype(F64)
    return (p - onehot) / B


def dice_sums(pred, target):
    """nn_dice_loss_sums.hlsl:25-54: per-sample (Σp·t, Σp, Σt)."""
    B = pred.shape[0]
    p = _f64(pred).reshape(B, -1)
    t = _f64(target).reshape(B, -1)
    return np.stack([(p * t).sum(1), p.sum(1), t.sum(1)], axis=1)


def dice_loss(pred, target):
    """nn_dice_loss.hlsl:52-55: 1 − 2I/(Σp+Σt+1e-6), per sample."""
    s = dice_sums(pred, target)
    return 1.0 - 2.0 * s[:, 0] / (s[:, 1] + s[:, 2] + 1e-6)


def dice_loss_grad(pred, target):
    """nn_dice_loss_grad.hlsl:22-33: dp = −2(t·D − I)/D² / B with
    D = Σp + Σt + 1e-6 (the incoming gradient is ignored, nn_engine.py:1303)."""
    B = pred.shape[0]
    s = dice_sums(pred, target)
    t = _f64(target).reshape(B, -1)
    D = (s[:, 1] + s[:, 2] + 1e-6)[:, None]
    g = -2.0 * (t * D - s[:, 0:1]) / (D * D) / B
    return g.reshape(pred.shape)


def argmax_correct(logits, labels):
    """nn_argmax_correct.hlsl:13-26: first-max-wins argmax (strict ``>``,
    starting from column 0) compared with uint(label).  Returns the count."""
    z = np.asarray(logits, dtype=np.float32)
    lab = np.asarray(labels, dtype=np.float32).reshape(-1).astype(np.int64)
    best = z[:, 0].copy()
    bi = np.zeros(z.shape[0], dtype=np.int64)
    for j in range(1, z.shape[1]):
        take = z[:, j] > best
        best = np.where(take, z[:, j], best)
        bi = np.where(take, j, bi)
    return int((bi == lab).sum())


# ----------------------------------------------------------------------------
# Optimisers and clipping
# ----------------------------------------------------------------------------

def sgd(w, g, lr, clip):
    """nn_sgd.hlsl:6-11: w −= lr·clamp(g, −clip, clip)."""
    g = np.clip(_f64(g), -clip, clip)
    return _f64(w) - lr * g


def grad_norm_scale(grads, max_norm):
    """grad_sq_reduce + grad_norm_final (nn_grad_sq_reduce.hlsl:20-30,
    nn_grad_norm_final.hlsl:22-35): norm = √Σg²; scale = max/(norm+1e-6) if
    norm > max else 1.  Same rule as clip_grad_norm (nn_engine.py:1335-1355)."""
    tot = 0.0
    for g in grads:
        g = _f64(g)
        tot += float((g * g).sum())
    norm = float(np.sqrt(tot))
    scale = max_norm / (norm + 1e-6) if norm > max_norm else 1.0
    return norm, scale


def sgd_clipped(w, g, lr, scale):
    """nn_sgd_clipped.hlsl:16-20: w −= lr·g·scale."""
    return _f64(w) - lr * _f64(g) * scale


def adam_step_size(lr, beta1, beta2, t):
    """Host-side bias correction of AdamW.step (nn_engine.py:2220)."""
    return lr * (1.0 - beta2 ** t) ** 0.5 / (1.0 - beta1 ** t)


def adam(w, g, m, v, step_size, beta1, beta2, eps, wd_eff, clip):
    """nn_adam.hlsl:20-33 with wd_eff = lr·weight_decay computed on the host
    (nn_engine.py:2235): element clip, moments, then
    w ← w − wd_eff·w − step·m/(√v + ε) using the *old* w for the decay."""
    g = np.clip(_f64(g), -clip, clip)
    w = _f64(w)
    m = beta1 * _f64(m) + (1.0 - beta1) * g
    v = beta2 * _f64(v) + (1.0 - beta2) * g * g
    w = w - wd_eff * w - step_size * m / (np.sqrt(v) + eps)
    return w, m, v
