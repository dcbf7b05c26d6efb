"""Float64 mini-autograd restating the backward semantics of nn_engine.py.

TEST INFRASTRUCTURE ONLY (see ``oracle/kernels.py``).  It reproduces, op by op,
what each reference ``Function.backward`` dispatches, so whole training steps of
the benchmark networks can be recomputed in float64 on the CPU:

* reverse-topological traversal seeded with ones (nn_engine.py:575-603);
* gradient accumulation = plain sums (nn_engine.py:605-610);
* per-op formulas from ``oracle.kernels`` with the reference's quirks kept:
  conv act==2 gets no tanh derivative (engine.cpp:816-835), BiasReLU masks on
  its *output* (nn_engine.py:1096), softmax-CE and Dice ignore the incoming
  gradient (nn_engine.py:1282-1288, :1303-1317), maxpool routes through the
  argmax indices (engine.cpp:906-930, summed deterministically).
"""
from __future__ import annotations

import numpy as np

from . import kernels as K

F64 = np.float64


class T:
    """A float64 tensor node.  ``data`` is float64; ``grad`` accumulates."""

    __slots__ = ("data", "grad", "requires_grad", "_parents", "_backward", "name", "pre", "own_idx")

    def __init__(self, data, requires_grad=False, name=None):
        self.data = np.asarray(data, dtype=F64)
        self.grad = None
        self.requires_grad = requires_grad
        self._parents = ()
        self._backward = None
        self.name = name
        self.pre = None       # pre-activation, when a decision pattern was given
        self.own_idx = None   # the oracle's own argmax scan (maxpool2d)

    @property
    def shape(self):
        return self.data.shape

    def _acc(self, g):
        """First gradient is kept, later ones are added with grad_accum
        (nn_engine.py:605-610)."""
        g = np.asarray(g, dtype=F64).reshape(self.data.shape)
        self.grad = g.copy() if self.grad is None else K.grad_accum(self.grad, g)

    def backward(self):
        topo, seen = [], set()
        stack = [(self, False)]
        while stack:
            v, done = stack.pop()
            if done:
                topo.append(v)
                continue
            if id(v) in seen:
                continue
            seen.add(id(v))
            stack.append((v, True))
            for p in v._parents:
                if p.requires_grad and id(p) not in seen:
                    stack.append((p, False))
        self.grad = np.ones_like(self.data)
        for v in reversed(topo):
            if v._backward is not None and v.grad is not None:
                v._backward(v.grad)


def _node(data, parents, backward):
    out = T(data, requires_grad=any(p.requires_grad for p in parents))
    if out.requires_grad:
        out._parents = tuple(parents)
        out._backward = backward
    return out


def conv2d(x, w, b, stride=1, padding=0, act=0, mask=None):
    """``mask`` (bool, output shape; act == 1 only) pins the ReLU decision
    (y > 0) to a given pattern, e.g. the device's own, so that a value
    within round-off of 0 cannot route the gradient differently.  The node
    then keeps the pre-activation as ``pre``, so that a caller can check the
    given decisions against the oracle's own (z > 0)."""
    z = None
    if act == 1 and mask is not None:
        z = K.conv_forward(x.data, w.data, b.data, stride, padding, 0)
        y = np.where(mask, z, 0.0)
    else:
        y = K.conv_forward(x.data, w.data, b.data, stride, padding, act)

    def bw(g):
        if act == 1 and mask is not None:
            g, y_mask, a = np.where(mask, g, 0.0), None, 0
        else:
            y_mask, a = y, act
        dW, db, dX = K.conv_backward(g, y_mask, x.data, w.data, stride, padding, a,
                                     need_x=x.requires_grad, need_w=w.requires_grad,
                                     need_b=b.requires_grad)
        if w.requires_grad:
            w._acc(dW)
        if b.requires_grad:
            b._acc(db)
        if x.requires_grad:
            x._acc(dX)
    node = _node(y, (x, w, b), bw)
    node.pre = z
    return node


def maxpool2d(x, pool_size=2, stride=2, indices=None):
    """``indices`` may be supplied (uint32, from the device) so that routing
    follows exactly the same argmax as the run under test; the node keeps the
    oracle's own scan as ``own_idx``."""
    out, idx = K.maxpool_forward(x.data, pool_size, stride)
    own_idx = idx
    if indices is not None:
        idx = np.asarray(indices, dtype=np.uint32).reshape(idx.shape)
        flat = x.data.reshape(-1)
        out = np.where(idx == K.IDX_NONE, -1e30, flat[np.minimum(idx, flat.size - 1).astype(np.int64)])

    def bw(g):
        x._acc(K.maxpool_backward(g, idx, x.data.size))
    node = _node(out, (x,), bw)
    node.name = idx
    node.own_idx = own_idx
    return node


def flatten(x):
    B = x.data.shape[0]

    def bw(g):
        x._acc(g)
    return _node(x.data.reshape(B, -1), (x,), bw)


def matmul(A, Bm, transA=False, transB=False):
    a = A.data.T if transA else A.data
    bm = Bm.data.T if transB else Bm.data

    def bw(g):
        if A.requires_grad:
            ga = g @ bm.T
            A._acc(ga.T if transA else ga)
        if Bm.requires_grad:
            gb = a.T @ g
            Bm._acc(gb.T if transB else gb)
    return _node(a @ bm, (A, Bm), bw)


def add_bias(A, b):
    def bw(g):
        if A.requires_grad:
            A._acc(g)
        if b.requires_grad:
            b._acc(g.sum(axis=0))
    return _node(K.add_bias(A.data, b.data), (A, b), bw)


def bias_relu(A, b, mask=None):
    """``mask`` pins the decision A + b > 0; the node keeps A + b as ``pre``."""
    out = K.bias_relu(A.data, b.data)
    pre = None
    if mask is not None:
        pre = K.add_bias(A.data, b.data)
        out = np.where(mask, pre, 0.0)

    def bw(g):
        eff = K.relu_grad(g, out) if mask is None else np.where(mask, g, 0.0)
        if A.requires_grad:
            A._acc(eff)
        if b.requires_grad:
            b._acc(eff.sum(axis=0))
    node = _node(out, (A, b), bw)
    node.pre = pre
    return node


def relu(x, mask=None):
    """``mask`` (bool) pins the decision x > 0 (see conv2d)."""
    if mask is None:
        def bw(g):
            x._acc(K.relu_grad(g, x.data))
        return _node(K.relu(x.data), (x,), bw)

    def bwm(g):
        x._acc(np.where(mask, g, 0.0))
    return _node(np.where(mask, x.data, 0.0), (x,), bwm)


def relu6(x, mask=None):
    """``mask`` (bool) pins the decision 0 < x < 6."""
    if mask is None:
        def bw(g):
            x._acc(K.relu6_grad(g, x.data))
        return _node(K.relu6(x.data), (x,), bw)

    def bwm(g):
        x._acc(np.where(mask, g, 0.0))
    return _node(np.where(mask, x.data, np.where(x.data >= 6.0, 6.0, 0.0)), (x,), bwm)


def sigmoid(x):
    y = K.sigmoid(x.data)

    def bw(g):
        x._acc(K.sigmoid_grad(g, y))
    return _node(y, (x,), bw)


def leaky_relu(x, alpha=0.1):
    def bw(g):
        x._acc(K.leaky_relu_grad(g, x.data, alpha))
    return _node(K.leaky_relu(x.data, alpha), (x,), bw)


def add(A, Bm):
    def bw(g):
        if A.requires_grad:
            A._acc(g)
        if Bm.requires_grad:
            Bm._acc(g)
    return _node(K.add(A.data, Bm.data), (A, Bm), bw)


def upsample2d(x, sH=2, sW=2):
    def bw(g):
        x._acc(K.upsample_backward(g, x.data.shape, sH, sW))
    return _node(K.upsample(x.data, sH, sW), (x,), bw)


def concat(ts):
    offs, o = [], 0
    for t in ts:
        offs.append(o)
        o += t.data.shape[1]

    def bw(g):
        for t, off in zip(ts, offs):
            if t.requires_grad:
                t._acc(K.slice_channels(g, off, t.data.shape[1]))
    return _node(K.concat([t.data for t in ts]), tuple(ts), bw)


def depthwise_conv2d(x, f, b, stride=1, padding=0):
    def bw(g):
        if x.requires_grad:
            x._acc(K.depthwise_backward_input(g, f.data, x.data.shape, stride, padding))
        if f.requires_grad or b.requires_grad:
            df, db = K.depthwise_backward_filter(g, x.data, f.data.shape[2], f.data.shape[3], stride, padding)
            if f.requires_grad:
                f._acc(df)
            if b.requires_grad:
                b._acc(db)
    return _node(K.depthwise_forward(x.data, f.data, b.data, stride, padding), (x, f, b), bw)


def global_avg_pool2d(x):
    def bw(g):
        x._acc(K.global_avg_pool_backward(g, x.data.shape))
    return _node(K.global_avg_pool(x.data), (x,), bw)


def batchnorm2d(x, gamma, beta, rm=None, rv=None, eps=1e-5, momentum=0.1):
    """Training-mode BN (BatchNorm2dFunc, nn_engine.py:1794-1868).  Returns
    (out, new_running_mean, new_running_var)."""
    mean, var, nrm, nrv = K.batchnorm_mean_var(x.data, rm, rv, momentum, True)
    y = K.batchnorm_forward(x.data, mean, var, gamma.data, beta.data, eps)

    def bw(g):
        dg, db = K.batchnorm_backward_reduce(x.data, g, mean, var, eps)
        if gamma.requires_grad:
            gamma._acc(dg)
        if beta.requires_grad:
            beta._acc(db)
        if x.requires_grad:
            x._acc(K.batchnorm_backward_dx(x.data, g, mean, var, gamma.data, dg, db, eps))
    return _node(y, (x, gamma, beta), bw), nrm, nrv


def softmax_ce(x, labels):
    p = K.softmax(x.data)
    loss = K.ce_loss(x.data, labels)

    def bw(g):
        x._acc(K.softmax_ce_grad(p, labels))
    out = _node(np.array([loss]), (x,), bw)
    return out


def dice_loss(pred, target):
    def bw(g):
        pred._acc(K.dice_loss_grad(pred.data, target))
    return _node(K.dice_loss(pred.data, target), (pred,), bw)
