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
