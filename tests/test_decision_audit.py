"""CPU tests of the decision audit (tests/workloads.py DecisionAudit) that the
whole-step GPU tests run on every ReLU / ReLU6 mask and max-pool argmax the
oracle adopts from the device.  Mistakes are planted in stand-in "device"
values built on the CPU from the oracle's own forward: a decision flipped far
from a tie, or a forward value that is off, must fail the check; a flip at a
genuine near-tie must pass."""
import numpy as np
import pytest

from oracle import kernels as K
from tests import workloads as WL
from tests.helpers import rng


def _conv_case():
    r = rng(90)
    x = r.standard_normal((2, 3, 9, 9))
    x[1] = 0.0                                 # image 1: z = bias exactly
    P = {"c.w": (0.3 * r.standard_normal((4, 3, 3, 3))).astype(np.float32),
         "c.b": np.array([1e-9, 0.2, -0.3, 0.5], np.float32)}
    z = K.conv_forward(x, P["c.w"], P["c.b"], 1, 1, 0)
    return x, P, z


def _run_conv(x, P, dev):
    ob = WL.Oracle(P, decisions=[("pos", dev)])
    ob.conv(ob.input(x), "c", 1, 1, act=1)
    return ob.audit


def test_exact_decisions_pass():
    x, P, z = _conv_case()
    dev = np.maximum(z, 0).astype(np.float32)
    audit = _run_conv(x, P, dev)
    msg = audit.check()
    assert "0 disagreements" in msg


def test_flipped_positive_output_is_caught():
    """A device forward that zeroes a clearly positive output (e.g. a tile
    its split-K finish skipped) must fail, although the adopted mask makes
    the oracle's loss and gradients agree with it."""
    x, P, z = _conv_case()
    dev = np.maximum(z, 0).astype(np.float32)
    i = np.unravel_index(np.argmax(z), z.shape)
    dev[i] = 0.0
    with pytest.raises(AssertionError, match="disagreements"):
        _run_conv(x, P, dev).check()


def test_near_tie_flip_passes():
    """Image 1 is all zeros, so its channel-0 outputs equal the bias 1e-9:
    a device that calls them non-positive disagrees only at a near-tie."""
    x, P, z = _conv_case()
    dev = np.maximum(z, 0).astype(np.float32)
    dev[1, 0] = 0.0
    audit = _run_conv(x, P, dev)
    assert "disagreements" in audit.check()
    assert audit.sites[0][2] == dev[1, 0].size


def test_wrong_forward_value_is_caught():
    x, P, z = _conv_case()
    dev = np.maximum(z, 0).astype(np.float32)
    i = np.unravel_index(np.argmax(z), z.shape)
    dev[i] *= 1.001                             # still positive, but off by 1e-3
    with pytest.raises(AssertionError, match="forward error"):
        _run_conv(x, P, dev).check()


def test_relu6_and_relu_inputs():
    r = rng(91)
    x = 4 * r.standard_normal((3, 50))
    for kind, fn in (("six", "relu6"), ("pos", "relu")):
        ob = WL.Oracle({}, decisions=[(kind, x.astype(np.float32))])
        getattr(ob, fn)(ob.input(x))
        ob.audit.check()
        bad = x.astype(np.float32)
        j = int(np.argmax(np.abs(x - 3.0) < 1.0))        # a value near 3, inside (0, 6)
        bad[np.unravel_index(j, x.shape)] = 7.0 if kind == "six" else -1.0
        ob = WL.Oracle({}, decisions=[(kind, bad)])
        getattr(ob, fn)(ob.input(x))
        with pytest.raises(AssertionError):
            ob.audit.check()


def test_pool_index_flip_is_caught_unless_tied():
    r = rng(92)
    x = r.standard_normal((1, 2, 6, 6))
    x[0, 1, 0, 0] = x[0, 1, 0, 1] = 5.0          # a genuine tie in window (0, 0) of plane 1
    _, own = K.maxpool_forward(x, 2, 2)
    ob = WL.Oracle({}, pool_indices=[own.copy()])
    ob.maxpool(ob.input(x), 2, 2)
    assert "0 disagreements" in ob.audit.check()
    tied = own.copy()
    tied[0, 1, 0, 0] = 1 * 36 + 1                 # the other 5.0 of the tie
    ob = WL.Oracle({}, pool_indices=[tied])
    ob.maxpool(ob.input(x), 2, 2)
    assert "1 disagreements" in ob.audit.check()
    wrong = own.copy()
    w0 = int(wrong[0, 0, 1, 1])
    wrong[0, 0, 1, 1] = next(i for i in (14, 15, 20, 21) if i != w0)  # not the window's max
    ob = WL.Oracle({}, pool_indices=[wrong])
    ob.maxpool(ob.input(x), 2, 2)
    with pytest.raises(AssertionError, match="margin"):
        ob.audit.check()
