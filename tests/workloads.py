"""Benchmark networks written once against a small op interface, runnable on
the device (drop-in ``nn_engine`` API) and on the float64 oracle
(``oracle.engine64``), so whole training steps can be compared.

Networks (the benchmark configurations):
  lenet     LeNet-5: conv 1->6 k5 +ReLU, maxpool 2, conv 6->16 k5 +ReLU, maxpool 2,
            Linear 256->120->84->10 (train_lenet.py:22-45 without BN)
  alexnet   AlexNet-224 with Linear 9216->4096->4096->1000 (train_alexnet.py:28-52)
  unet      UNet-base16: 4 levels of conv3x3-BN-ReLU x2, maxpool 2, nearest
            upsample x2 + channel concat, 1x1 head, sigmoid, Dice loss
  mobilenet MobileNetV2 inverted-residual stack 16->24 s2, 24->24, 24->32 s2,
            32->32 x2 (expand x6, BN, ReLU6, depthwise 3x3, BN, ReLU6, 1x1
            project, BN, residual add when s == 1 and Cin == Cout), then
            global average pool + Linear -> 10 + softmax-CE
"""
from __future__ import annotations

import numpy as np


# ------------------------------------------------------------------ params
def conv_p(rng, P, name, cin, cout, k, bias=True):
    P[name + ".w"] = (rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
    P[name + ".b"] = (0.01 * rng.standard_normal(cout)).astype(np.float32) if bias else np.zeros(cout, np.float32)


def lin_p(rng, P, name, fin, fout):
    P[name + ".w"] = (rng.standard_normal((fin, fout)) * np.sqrt(2.0 / fin)).astype(np.float32)
    P[name + ".b"] = (0.01 * rng.standard_normal(fout)).astype(np.float32)


def bn_p(rng, P, name, c):
    P[name + ".g"] = (1 + 0.1 * rng.standard_normal(c)).astype(np.float32)
    P[name + ".be"] = (0.1 * rng.standard_normal(c)).astype(np.float32)


def dw_p(rng, P, name, c, k):
    P[name + ".w"] = (rng.standard_normal((c, 1, k, k)) * np.sqrt(2.0 / (k * k))).astype(np.float32)
    P[name + ".b"] = (0.01 * rng.standard_normal(c)).astype(np.float32)


# ------------------------------------------------------------------ backends
class Device:
    """Ops through the drop-in nn_engine module."""

    def __init__(self, nn, params):
        self.nn = nn
        self.P = {k: nn.Tensor(v.copy(), requires_grad=True, track=False) for k, v in params.items()}
        self.rs = {}
        self.pool_nodes = []
        self.mask_nodes = []  # (tensor, kind) of every ReLU-type decision, in order

    def input(self, a):
        return self.nn.Tensor(a, track=True)

    def conv(self, x, name, s=1, p=0, act=0):
        y = self.nn.conv2d(x, self.P[name + ".w"], self.P[name + ".b"], s, p, act)
        if act == 1:
            self.mask_nodes.append((y, "pos"))
        return y

    def maxpool(self, x, k, s):
        y = self.nn.maxpool2d(x, k, s)
        self.pool_nodes.append(y)
        return y

    def relu(self, x):
        self.mask_nodes.append((x, "pos"))
        return self.nn.relu(x)

    def relu6(self, x):
        self.mask_nodes.append((x, "six"))
        return self.nn.relu6(x)

    def sigmoid(self, x):
        return self.nn.sigmoid(x)

    def flatten(self, x):
        return self.nn.flatten(x)

    def linear(self, x, name, relu):
        m = self.nn.matmul(x, self.P[name + ".w"])
        if relu:
            y = self.nn.bias_relu(m, self.P[name + ".b"])
            self.mask_nodes.append((y, "pos"))
            return y
        return self.nn.add_bias(m, self.P[name + ".b"])

    def bn(self, x, name):
        c = x.shape[1]
        if name not in self.rs:
            self.rs[name] = (self.nn.Tensor(np.zeros(c, np.float32), track=False),
                             self.nn.Tensor(np.ones(c, np.float32), track=False))
        rm, rv = self.rs[name]
        return self.nn.batchnorm2d(x, self.P[name + ".g"], self.P[name + ".be"], rm, rv)

    def upsample(self, x):
        return self.nn.upsample2d(x, 2, 2)

    def concat(self, ts):
        return self.nn.concat(ts)

    def add(self, a, b):
        return self.nn.add(a, b)

    def dwconv(self, x, name, s, p):
        return self.nn.depthwise_conv2d(x, self.P[name + ".w"], self.P[name + ".b"], s, p)

    def gap(self, x):
        return self.nn.global_avg_pool2d(x)

    def softmax_ce(self, z, labels):
        return self.nn.softmax_ce(z, self.nn.Tensor(labels, track=True))

    def dice(self, p, target):
        return self.nn.dice_loss(p, self.nn.Tensor(target, track=True))

    def pool_indices(self):
        """uint32 argmax indices of every maxpool of the last forward, read
        before the backward consumes them."""
        out = []
        for y in self.pool_nodes:
            h = y._ctx.indices_handle
            t = self.nn.Tensor.from_gpu(h, y.shape, track=False)
            idx = t.sync().copy().view(np.uint32)
            t.gpu_buf = None  # the Function still owns the handle
            out.append(idx)
        return out

    def masks(self):
        """The device's ReLU-type decisions of the last forward (bool arrays,
        in op order): y > 0 for conv+ReLU and bias+ReLU outputs, x > 0 for
        relu inputs, 0 < x < 6 for relu6 inputs."""
        out = []
        for t, kind in self.mask_nodes:
            v = t.sync().copy()
            out.append((v > 0) & (v < 6) if kind == "six" else v > 0)
        return out

    def grads(self):
        return {k: v.grad.sync().copy() for k, v in self.P.items() if v.grad is not None}

    def values(self):
        return {k: v.sync().copy() for k, v in self.P.items()}


class Oracle:
    """The same ops on the float64 oracle.  `pool_indices` (from the device
    run) pins maxpool routing to the argmax the device chose."""

    def __init__(self, params, pool_indices=None, masks=None):
        from oracle import engine64 as E
        self.E = E
        self.P = {k: E.T(v, requires_grad=True) for k, v in params.items()}
        self.pool_indices = list(pool_indices) if pool_indices is not None else None
        self.masks = list(masks) if masks is not None else None
        self.rs = {}

    def _mask(self):
        return self.masks.pop(0) if self.masks else None

    def input(self, a):
        return self.E.T(a)

    def conv(self, x, name, s=1, p=0, act=0):
        return self.E.conv2d(x, self.P[name + ".w"], self.P[name + ".b"], s, p, act,
                             mask=self._mask() if act == 1 else None)

    def maxpool(self, x, k, s):
        idx = self.pool_indices.pop(0) if self.pool_indices else None
        return self.E.maxpool2d(x, k, s, indices=idx)

    def relu(self, x):
        return self.E.relu(x, mask=self._mask())

    def relu6(self, x):
        return self.E.relu6(x, mask=self._mask())

    def sigmoid(self, x):
        return self.E.sigmoid(x)

    def flatten(self, x):
        return self.E.flatten(x)

    def linear(self, x, name, relu):
        m = self.E.matmul(x, self.P[name + ".w"])
        if relu:
            return self.E.bias_relu(m, self.P[name + ".b"], mask=self._mask())
        return self.E.add_bias(m, self.P[name + ".b"])

    def bn(self, x, name):
        c = x.data.shape[1]
        rm, rv = self.rs.get(name, (np.zeros(c), np.ones(c)))
        y, nrm, nrv = self.E.batchnorm2d(x, self.P[name + ".g"], self.P[name + ".be"], rm, rv)
        self.rs[name] = (nrm, nrv)
        return y

    def upsample(self, x):
        return self.E.upsample2d(x, 2, 2)

    def concat(self, ts):
        return self.E.concat(ts)

    def add(self, a, b):
        return self.E.add(a, b)

    def dwconv(self, x, name, s, p):
        return self.E.depthwise_conv2d(x, self.P[name + ".w"], self.P[name + ".b"], s, p)

    def gap(self, x):
        return self.E.global_avg_pool2d(x)

    def softmax_ce(self, z, labels):
        return self.E.softmax_ce(z, labels)

    def dice(self, p, target):
        return self.E.dice_loss(p, target)

    def grads(self):
        return {k: v.grad for k, v in self.P.items() if v.grad is not None}


# ------------------------------------------------------------------ networks
def lenet_params(rng):
    P = {}
    conv_p(rng, P, "c1", 1, 6, 5)
    conv_p(rng, P, "c2", 6, 16, 5)
    lin_p(rng, P, "l1", 256, 120)
    lin_p(rng, P, "l2", 120, 84)
    lin_p(rng, P, "l3", 84, 10)
    return P


def lenet(be, x):
    h = be.maxpool(be.conv(be.input(x), "c1", act=1), 2, 2)
    h = be.maxpool(be.conv(h, "c2", act=1), 2, 2)
    h = be.flatten(h)
    h = be.linear(h, "l1", True)
    h = be.linear(h, "l2", True)
    return be.linear(h, "l3", False)


ALEX = [("c1", 3, 64, 11, 4, 2), ("c2", 64, 192, 5, 1, 2), ("c3", 192, 384, 3, 1, 1),
        ("c4", 384, 256, 3, 1, 1), ("c5", 256, 256, 3, 1, 1)]


def alexnet_params(rng):
    P = {}
    for n, ci, co, k, _, _ in ALEX:
        conv_p(rng, P, n, ci, co, k)
    lin_p(rng, P, "l1", 9216, 4096)
    lin_p(rng, P, "l2", 4096, 4096)
    lin_p(rng, P, "l3", 4096, 1000)
    return P


def alexnet(be, x):
    h = be.input(x)
    for n, _, _, _, s, p in ALEX:
        h = be.conv(h, n, s, p, act=1)
        if n in ("c1", "c2", "c5"):
            h = be.maxpool(h, 3, 2)
    h = be.flatten(h)
    h = be.linear(h, "l1", True)
    h = be.linear(h, "l2", True)
    return be.linear(h, "l3", False)


def unet_params(rng, base=16, levels=4, cin=3):
    P = {}
    ch = [base * 2 ** i for i in range(levels)]
    prev = cin
    for i, c in enumerate(ch):
        conv_p(rng, P, f"e{i}a", prev, c, 3)
        bn_p(rng, P, f"e{i}a.bn", c)
        conv_p(rng, P, f"e{i}b", c, c, 3)
        bn_p(rng, P, f"e{i}b.bn", c)
        prev = c
    cb = base * 2 ** levels
    conv_p(rng, P, "ba", prev, cb, 3)
    bn_p(rng, P, "ba.bn", cb)
    conv_p(rng, P, "bb", cb, cb, 3)
    bn_p(rng, P, "bb.bn", cb)
    prev = cb
    for i in reversed(range(levels)):
        c = ch[i]
        conv_p(rng, P, f"d{i}a", prev + c, c, 3)
        bn_p(rng, P, f"d{i}a.bn", c)
        conv_p(rng, P, f"d{i}b", c, c, 3)
        bn_p(rng, P, f"d{i}b.bn", c)
        prev = c
    conv_p(rng, P, "head", prev, 1, 1)
    return P


def _cbr(be, h, name):
    return be.relu(be.bn(be.conv(h, name, 1, 1), name + ".bn"))


def unet(be, x, levels=4):
    h = be.input(x)
    skips = []
    for i in range(levels):
        h = _cbr(be, _cbr(be, h, f"e{i}a"), f"e{i}b")
        skips.append(h)
        h = be.maxpool(h, 2, 2)
    h = _cbr(be, _cbr(be, h, "ba"), "bb")
    for i in reversed(range(levels)):
        h = be.concat([be.upsample(h), skips[i]])
        h = _cbr(be, _cbr(be, h, f"d{i}a"), f"d{i}b")
    return be.sigmoid(be.conv(h, "head", 1, 0))


MBV2 = [(16, 24, 2), (24, 24, 1), (24, 32, 2), (32, 32, 1), (32, 32, 1)]


def mobilenet_params(rng, ncls=10):
    P = {}
    for i, (ci, co, _) in enumerate(MBV2):
        h = ci * 6
        conv_p(rng, P, f"b{i}.exp", ci, h, 1)
        bn_p(rng, P, f"b{i}.bn1", h)
        dw_p(rng, P, f"b{i}.dw", h, 3)
        bn_p(rng, P, f"b{i}.bn2", h)
        conv_p(rng, P, f"b{i}.proj", h, co, 1)
        bn_p(rng, P, f"b{i}.bn3", co)
    lin_p(rng, P, "fc", MBV2[-1][1], ncls)
    return P


def mobilenet(be, x):
    h = be.input(x)
    for i, (ci, co, s) in enumerate(MBV2):
        t = be.relu6(be.bn(be.conv(h, f"b{i}.exp"), f"b{i}.bn1"))
        t = be.relu6(be.bn(be.dwconv(t, f"b{i}.dw", s, 1), f"b{i}.bn2"))
        t = be.bn(be.conv(t, f"b{i}.proj"), f"b{i}.bn3")
        h = be.add(t, h) if (s == 1 and ci == co) else t
    return be.linear(be.gap(h), "fc", False)


# ------------------------------------------------------------------ reference UNet run
# The 3-level UNet-base16 of compare_unet_20batch.py (conv3x3 + ReLU x2 per
# block, no BN), with the weights that script draws from RandomState(42).
UNET3_BLOCKS = [("enc1", 3, 16), ("enc2", 16, 32), ("enc3", 32, 64), ("bot", 64, 128),
                ("up3", 192, 64), ("up2", 96, 32), ("up1", 48, 16)]


def unet3_ref_params():
    rng = np.random.RandomState(42)
    P = {}
    for name, cin, cout in UNET3_BLOCKS:
        P[name + ".w1"] = rng.randn(cout, cin, 3, 3).astype(np.float32) * np.sqrt(2.0 / (cin * 9))
        P[name + ".b1"] = np.zeros(cout, np.float32)
        P[name + ".w2"] = rng.randn(cout, cout, 3, 3).astype(np.float32) * np.sqrt(2.0 / (cout * 9))
        P[name + ".b2"] = np.zeros(cout, np.float32)
    P["final.w"] = rng.randn(1, 16, 1, 1).astype(np.float32) * np.sqrt(2.0 / 16)
    P["final.b"] = np.zeros(1, np.float32)
    return P


def _block(be, h, name):
    h = be.relu(be.conv(h, name + "@1", 1, 1))
    return be.relu(be.conv(h, name + "@2", 1, 1))


def unet3_ref(be, x):
    e1 = _block(be, be.input(x), "enc1")
    e2 = _block(be, be.maxpool(e1, 2, 2), "enc2")
    e3 = _block(be, be.maxpool(e2, 2, 2), "enc3")
    b = _block(be, be.maxpool(e3, 2, 2), "bot")
    d3 = _block(be, be.concat([be.upsample(b), e3]), "up3")
    d2 = _block(be, be.concat([be.upsample(d3), e2]), "up2")
    d1 = _block(be, be.concat([be.upsample(d2), e1]), "up1")
    return be.sigmoid(be.conv(d1, "final@", 1, 0))


def unet3_rename(P):
    """Parameter names as the backends look them up: '<block>@1.w' etc."""
    out = {}
    for k, v in P.items():
        blk, kind = k.split(".")
        if blk == "final":
            out["final@." + kind] = v
        else:
            out[f"{blk}@{kind[1]}.{kind[0]}"] = v
    return out


def segment_batches(path):
    """(x, y) float32 batches of the golden segment fixture, in step order."""
    d = np.load(path)
    X = d["images_u8"].astype(np.float32).transpose(0, 3, 1, 2) / 255.0
    Y = np.unpackbits(d["masks"], axis=-1)[:, None, :, :].astype(np.float32)
    return [(X[2 * i:2 * i + 2], Y[2 * i:2 * i + 2]) for i in range(len(X) // 2)], d["dc_loss"], d["dc_norm"]
