"""Shared test helpers: error metric, host<->device helpers, seeded inputs."""
import ctypes

import numpy as np


def rel_err(got, ref):
    """max|got - ref| / max|ref| -- the reference's parity metric
    (test_backward_base16.py:205, nn_verify.py:242-243)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    den = np.max(np.abs(ref))
    num = np.max(np.abs(got - ref)) if got.size else 0.0
    if den == 0:
        return float(num)
    return float(num / den)


TOL = 1e-4  # max|g - g_ref| / max|g_ref| bound for every gradient tensor


def rng(seed):
    return np.random.default_rng(seed)


def upload(eng, arr):
    """Create a device buffer from a float32 array; returns the handle."""
    a = np.ascontiguousarray(arr, dtype=np.float32)
    h = eng.lib.CreateBuffer(a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), a.size)
    assert h, eng.last_error()
    return h


def download(eng, h, shape):
    out = np.empty(int(np.prod(shape)), dtype=np.float32)
    eng.lib.ReadBuffer(h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out.reshape(shape)


def release(eng, *hs):
    for h in hs:
        if h:
            eng.lib.ReleaseBuffer(h)


def he(r, shape, fan_in):
    return (r.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)
