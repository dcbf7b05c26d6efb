"""Float64 oracle versions of the benchmark networks (TEST INFRASTRUCTURE ONLY).

Each ``*_step`` runs one training step -- forward, loss, backward, optimiser --
with ``oracle.engine64`` on float64 copies of the given float32 parameters and
returns (loss, {name: grad}, {name: new_param}).  The graphs follow the
reference's training scripts:

* LeNet-5: train_lenet.py:22-45 without BN (conv 1->6 k5, pool, conv 6->16 k5,
  pool, Linear 256->120->84->10), ReLU fused in the conv (actType 1) as the
  benchmark configuration states; SGD with element clip.
* AlexNet-224: train_alexnet.py:28-52 with Linear 9216->4096->4096->1000;
  AdamW with element clip.
* Single conv layer backward (engine.cpp:802-878 on one layer).
"""
from __future__ import annotations

import numpy as np

from . import engine64 as E
from . import kernels as K

ALEXNET_CONVS = [  # name, inC, outC, k, stride, pad
    ("c1", 3, 64, 11, 4, 2),
    ("c2", 64, 192, 5, 1, 2),
    ("c3", 192, 384, 3, 1, 1),
    ("c4", 384, 256, 3, 1, 1),
    ("c5", 256, 256, 3, 1, 1),
]
ALEXNET_FCS = [("l1", 9216, 4096, True), ("l2", 4096, 4096, True), ("l3", 4096, 1000, False)]

LENET_CONVS = [("c1", 1, 6, 5, 1, 0), ("c2", 6, 16, 5, 1, 0)]
LENET_FCS = [("l1", 256, 120, True), ("l2", 120, 84, True), ("l3", 84, 10, False)]


def he_params(rng, convs, fcs):
    """He-normal weights (N(0, 2/fan_in)), zero biases; linear weights are
    (in, out) as in nn_engine.py:1876."""
    p = {}
    for name, cin, cout, k, _, _ in convs:
        p[name + ".w"] = (rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
        p[name + ".b"] = np.zeros(cout, np.float32)
    for name, fin, fout, _ in fcs:
        p[name + ".w"] = (rng.standard_normal((fin, fout)) * np.sqrt(2.0 / fin)).astype(np.float32)
        p[name + ".b"] = np.zeros(fout, np.float32)
    return p


def _forward_convnet(P, x, convs, fcs, pool_after, pool_k, pool_s, pool_indices=None):
    h = E.T(x)
    pi = 0
    for name, _, _, _, s, pad in convs:
        h = E.conv2d(h, P[name + ".w"], P[name + ".b"], s, pad, 1)
        if name in pool_after:
            idx = None if pool_indices is None else pool_indices[pi]
            h = E.maxpool2d(h, pool_k, pool_s, indices=idx)
            pi += 1
    h = E.flatten(h)
    for name, _, _, relu in fcs:
        m = E.matmul(h, P[name + ".w"])
        h = E.bias_relu(m, P[name + ".b"]) if relu else E.add_bias(m, P[name + ".b"])
    return h


def _grads(P):
    return {k: (v.grad if v.grad is not None else np.zeros_like(v.data)) for k, v in P.items()}


def lenet_step(params, x, labels, lr=0.01, clip=1.0, pool_indices=None):
    P = {k: E.T(v, requires_grad=True) for k, v in params.items()}
    logits = _forward_convnet(P, x, LENET_CONVS, LENET_FCS, ("c1", "c2"), 2, 2, pool_indices)
    loss = E.softmax_ce(logits, labels)
    loss.backward()
    g = _grads(P)
    new = {k: K.sgd(params[k], g[k], lr, clip) for k in params}
    return float(loss.data[0]), g, new


def alexnet_step(params, x, labels, t=1, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, wd=0.01, clip=1.0,
                 m=None, v=None, pool_indices=None):
    P = {k: E.T(v_, requires_grad=True) for k, v_ in params.items()}
    logits = _forward_convnet(P, x, ALEXNET_CONVS, ALEXNET_FCS, ("c1", "c2", "c5"), 3, 2, pool_indices)
    loss = E.softmax_ce(logits, labels)
    loss.backward()
    g = _grads(P)
    step = K.adam_step_size(lr, betas[0], betas[1], t)
    new, nm, nv = {}, {}, {}
    for k in params:
        m0 = np.zeros(params[k].shape) if m is None else m[k]
        v0 = np.zeros(params[k].shape) if v is None else v[k]
        new[k], nm[k], nv[k] = K.adam(params[k], g[k], m0, v0, step, betas[0], betas[1], eps, lr * wd, clip)
    return float(loss.data[0]), g, new, nm, nv


def conv_backward_step(x, w, dy, stride=1, pad=1):
    """One ReLU conv layer's backward (engine.cpp:802-878): the forward output
    y = ReLU(conv(x, w)) sets the mask, then dW, db and dX."""
    y = K.conv_forward(x, w, np.zeros(w.shape[0]), stride, pad, 1)
    return K.conv_backward(dy, y, x, w, stride, pad, 1)


MBV2_BLOCKS = [(16, 24, 2), (24, 24, 1), (24, 32, 2), (32, 32, 1), (32, 32, 1)]


def mobilenet_stack_params(rng, ncls=10):
    """Inverted-residual stack (expand x6, BN, ReLU6, depthwise 3x3, BN, ReLU6,
    1x1 project, BN) + GAP + Linear; He weights, BN gamma 1 / beta 0."""
    P = {}
    for i, (ci, co, _) in enumerate(MBV2_BLOCKS):
        h = ci * 6
        P[f"b{i}.exp.w"] = (rng.standard_normal((h, ci, 1, 1)) * np.sqrt(2.0 / ci)).astype(np.float32)
        P[f"b{i}.dw.w"] = (rng.standard_normal((h, 1, 3, 3)) * np.sqrt(2.0 / 9)).astype(np.float32)
        P[f"b{i}.proj.w"] = (rng.standard_normal((co, h, 1, 1)) * np.sqrt(2.0 / h)).astype(np.float32)
        for n, c in (("exp", h), ("dw", h), ("proj", co)):
            P[f"b{i}.{n}.b"] = np.zeros(c, np.float32)
        for n, c in (("bn1", h), ("bn2", h), ("bn3", co)):
            P[f"b{i}.{n}.g"] = np.ones(c, np.float32)
            P[f"b{i}.{n}.be"] = np.zeros(c, np.float32)
    P["fc.w"] = (rng.standard_normal((MBV2_BLOCKS[-1][1], ncls)) * np.sqrt(2.0 / MBV2_BLOCKS[-1][1])).astype(np.float32)
    P["fc.b"] = np.zeros(ncls, np.float32)
    return P


def mobilenet_stack_step(params, x, labels, lr=0.01):
    """Forward (BN in training mode), softmax-CE, backward, SGD without
    element clip (clip 1e30)."""
    P = {k: E.T(v, requires_grad=True) for k, v in params.items()}
    h = E.T(x)
    for i, (ci, co, s) in enumerate(MBV2_BLOCKS):
        bn = lambda t, n: E.batchnorm2d(t, P[f"b{i}.{n}.g"], P[f"b{i}.{n}.be"])[0]
        t = E.relu6(bn(E.conv2d(h, P[f"b{i}.exp.w"], P[f"b{i}.exp.b"]), "bn1"))
        t = E.relu6(bn(E.depthwise_conv2d(t, P[f"b{i}.dw.w"], P[f"b{i}.dw.b"], s, 1), "bn2"))
        t = bn(E.conv2d(t, P[f"b{i}.proj.w"], P[f"b{i}.proj.b"]), "bn3")
        h = E.add(t, h) if (s == 1 and ci == co) else t
    loss = E.softmax_ce(E.add_bias(E.matmul(E.global_avg_pool2d(h), P["fc.w"]), P["fc.b"]), labels)
    loss.backward()
    g = _grads(P)
    return float(loss.data[0]), g, {k: K.sgd(params[k], g[k], lr, 1e30) for k in params}


def unet_params(rng, base=16, levels=4, cin=3):
    """UNet with conv3x3-BN-ReLU x2 per level (He weights, zero biases)."""
    P = {}

    def cbr(name, ci, co):
        P[name + ".w"] = (rng.standard_normal((co, ci, 3, 3)) * np.sqrt(2.0 / (ci * 9))).astype(np.float32)
        P[name + ".b"] = np.zeros(co, np.float32)
        P[name + ".g"] = np.ones(co, np.float32)
        P[name + ".be"] = np.zeros(co, np.float32)
    ch = [base * 2 ** i for i in range(levels)]
    prev = cin
    for i, c in enumerate(ch):
        cbr(f"e{i}a", prev, c)
        cbr(f"e{i}b", c, c)
        prev = c
    cb = base * 2 ** levels
    cbr("ba", prev, cb)
    cbr("bb", cb, cb)
    prev = cb
    for i in reversed(range(levels)):
        cbr(f"d{i}a", prev + ch[i], ch[i])
        cbr(f"d{i}b", ch[i], ch[i])
        prev = ch[i]
    P["head.w"] = (rng.standard_normal((1, prev, 1, 1)) * np.sqrt(2.0 / prev)).astype(np.float32)
    P["head.b"] = np.zeros(1, np.float32)
    return P


def unet_step(params, x, target, levels=4, lr=1e-3, max_norm=1.0):
    """Forward, Dice on the sigmoid output, backward, global-norm clip, Adam
    (first step)."""
    P = {k: E.T(v, requires_grad=True) for k, v in params.items()}

    def cbr(h, n):
        c = E.conv2d(h, P[n + ".w"], P[n + ".b"], 1, 1)
        return E.relu(E.batchnorm2d(c, P[n + ".g"], P[n + ".be"])[0])
    h = E.T(x)
    skips = []
    for i in range(levels):
        h = cbr(cbr(h, f"e{i}a"), f"e{i}b")
        skips.append(h)
        h = E.maxpool2d(h, 2, 2)
    h = cbr(cbr(h, "ba"), "bb")
    for i in reversed(range(levels)):
        h = cbr(cbr(E.concat([E.upsample2d(h, 2, 2), skips[i]]), f"d{i}a"), f"d{i}b")
    loss = E.dice_loss(E.sigmoid(E.conv2d(h, P["head.w"], P["head.b"])), target)
    loss.backward()
    g = _grads(P)
    names = sorted(g)
    _, scale = K.grad_norm_scale([g[k] for k in names], max_norm)
    step = K.adam_step_size(lr, 0.9, 0.999, 1)
    new = {}
    for k in params:
        z = np.zeros(params[k].shape)
        new[k] = K.adam(params[k], g[k] * scale, z, z, step, 0.9, 0.999, 1e-8, 0.0, 1e30)[0]
    return float(np.mean(loss.data)), g, new
