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


# ------------------------------------------------------------------ decisions
class DecisionAudit:
    """Checks the discrete decisions the oracle adopts from the device run.

    The oracle routes gradients through the device's ReLU / ReLU6 masks and
    max-pool argmax indices, so that an activation within float32 round-off
    of 0, 6 or a tie cannot send a gradient down another path than the one
    under test.  Adoption alone would also hide a wrong forward (a positive
    output zeroed by the device would be zeroed by the oracle too), so every
    adopted decision is compared with the oracle's own:

    * ReLU (conv + ReLU, bias + ReLU, relu on its input): own = z > 0, where
      z is the oracle's float64 pre-activation; a disagreement must be a
      near-tie, |z| <= tie_tol * max|z| of that tensor;
    * ReLU6: own = 0 < z < 6; near-tie: min(|z|, |z - 6|) <= tie_tol * max|z|;
    * max-pool: own = the oracle's first-max scan; near-tie: the input values
      at the two indices differ by <= tie_tol * max|x|.

    It also compares the device's forward values with the oracle's: the
    device's ReLU-type outputs where both sides call them positive, and the
    device's relu / relu6 inputs everywhere, relative to max|z| (fwd_tol)."""

    def __init__(self):
        self.sites = []   # (kind, elements, disagreements, worst tie margin, forward error)

    @staticmethod
    def _rel(a, scale):
        return float(a) / scale if scale > 0 else float(a)

    def relu(self, kind, z, dev, dev_is_output):
        """kind "pos" or "six"; z: oracle pre-activation; dev: the device's
        values (the ReLU output when dev_is_output, else its input)."""
        z = np.asarray(z, np.float64)
        dev = np.asarray(dev, np.float64).reshape(z.shape)
        scale = float(np.max(np.abs(z))) if z.size else 0.0
        if kind == "six":
            mine, theirs = (z > 0) & (z < 6), (dev > 0) & (dev < 6)
            margin = np.minimum(np.abs(z), np.abs(z - 6.0))
        else:
            mine, theirs = z > 0, dev > 0
            margin = np.abs(z)
        flips = mine != theirs
        worst = self._rel(margin[flips].max(), scale) if flips.any() else 0.0
        both = (mine & theirs) if dev_is_output else np.ones(z.shape, bool)
        ferr = self._rel(np.abs(dev[both] - z[both]).max(), scale) if both.any() else 0.0
        self.sites.append((kind, z.size, int(flips.sum()), worst, ferr))

    def pool(self, x, own_idx, dev_idx):
        x = np.asarray(x, np.float64).reshape(-1)
        own = np.asarray(own_idx, np.uint32).reshape(-1)
        dev = np.asarray(dev_idx, np.uint32).reshape(-1)
        flips = own != dev
        worst = 0.0
        if flips.any():
            scale = float(np.max(np.abs(x)))
            n = x.size
            a, b = own[flips].astype(np.int64), dev[flips].astype(np.int64)
            if (a >= n).any() or (b >= n).any():      # one side found no maximum
                worst = float("inf")
            else:
                worst = self._rel(np.abs(x[a] - x[b]).max(), scale)
        self.sites.append(("pool", own.size, int(flips.sum()), worst, 0.0))

    def check(self, tie_tol=1e-5, fwd_tol=1e-5):
        """Assert every disagreement is a near-tie and every forward value is
        close; returns a one-line summary (the counts) for the test log."""
        assert self.sites, "no decision was audited"
        flips = sum(s[2] for s in self.sites)
        n = sum(s[1] for s in self.sites)
        worst_tie = max(s[3] for s in self.sites)
        worst_fwd = max(s[4] for s in self.sites)
        msg = (f"{len(self.sites)} decision sites, {n} decisions, {flips} disagreements "
               f"(worst tie margin {worst_tie:.2e}), forward max rel err {worst_fwd:.2e}")
        for i, (kind, _, nf, tie, fe) in enumerate(self.sites):
            assert tie <= tie_tol, f"site {i} ({kind}): {nf} disagreements, margin {tie:.3e}; {msg}"
            assert fe <= fwd_tol, f"site {i} ({kind}): forward error {fe:.3e}; {msg}"
        return msg


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

    def decisions(self):
        """The device's values at every ReLU-type decision of the last forward,
        in op order, as (kind, float32 array): the outputs of conv + ReLU and
        bias + ReLU, the inputs of relu ("pos") and relu6 ("six").  The
        decision is v > 0 (0 < v < 6 for "six")."""
        return [(kind, t.sync().copy()) for t, kind in self.mask_nodes]

    def grads(self):
        return {k: v.grad.sync().copy() for k, v in self.P.items() if v.grad is not None}

    def values(self):
        return {k: v.sync().copy() for k, v in self.P.items()}


class Oracle:
    """The same ops on the float64 oracle.  `pool_indices` and `decisions`
    (from the device run: Device.pool_indices(), Device.decisions()) pin the
    max-pool routing and the ReLU / ReLU6 masks to the device's choices, and
    `audit` (a DecisionAudit) records each adopted decision against the
    oracle's own; call audit.check() after the forward."""

    def __init__(self, params, pool_indices=None, decisions=None):
        from oracle import engine64 as E
        self.E = E
        self.P = {k: E.T(v, requires_grad=True) for k, v in params.items()}
        self.pool_indices = list(pool_indices) if pool_indices is not None else None
        self.decisions = list(decisions) if decisions is not None else None
        self.audit = DecisionAudit()
        self.rs = {}

    def _decision(self, expect):
        if not self.decisions:
            return None, None
        kind, v = self.decisions.pop(0)
        assert kind == expect, (kind, expect)
        return v, ((v > 0) & (v < 6) if kind == "six" else v > 0)

    def input(self, a):
        return self.E.T(a)

    def conv(self, x, name, s=1, p=0, act=0):
        dev, mask = self._decision("pos") if act == 1 else (None, None)
        y = self.E.conv2d(x, self.P[name + ".w"], self.P[name + ".b"], s, p, act, mask=mask)
        if mask is not None:
            self.audit.relu("pos", y.pre, dev, dev_is_output=True)
        return y

    def maxpool(self, x, k, s):
        idx = self.pool_indices.pop(0) if self.pool_indices else None
        y = self.E.maxpool2d(x, k, s, indices=idx)
        if idx is not None:
            self.audit.pool(x.data, y.own_idx, idx)
        return y

    def relu(self, x):
        dev, mask = self._decision("pos")
        if mask is not None:
            self.audit.relu("pos", x.data, dev, dev_is_output=False)
        return self.E.relu(x, mask=mask)

    def relu6(self, x):
        dev, mask = self._decision("six")
        if mask is not None:
            self.audit.relu("six", x.data, dev, dev_is_output=False)
        return self.E.relu6(x, mask=mask)

    def sigmoid(self, x):
        return self.E.sigmoid(x)

    def flatten(self, x):
        return self.E.flatten(x)

    def linear(self, x, name, relu):
        m = self.E.matmul(x, self.P[name + ".w"])
        if relu:
            dev, mask = self._decision("pos")
            y = self.E.bias_relu(m, self.P[name + ".b"], mask=mask)
            if mask is not None:
                self.audit.relu("pos", y.pre, dev, dev_is_output=True)
            return y
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
