"""GPU parity of the memory-bound kernels (RunShader registry and fused entry
points) against the float64 oracle, plus the buffer API and the D3D11
out-of-bounds rules the reference relies on."""
import ctypes
import struct

import numpy as np
import pytest

from oracle import kernels as K
from tests.helpers import TOL, download, rel_err, release, rng, upload

pytestmark = pytest.mark.gpu


def fbits(f):
    return struct.unpack("I", struct.pack("f", f))[0]


def run(eng, name, srvs, uavs, *cb):
    """RunShader with the constant-buffer words given as ints."""
    ns, nu = len(srvs), len(uavs)
    sa = (ctypes.c_void_p * max(ns, 1))(*srvs)
    ua = (ctypes.c_void_p * max(nu, 1))(*uavs)
    th = (ctypes.c_uint * 3)(1, 1, 1)
    if cb:
        cba = (ctypes.c_uint * len(cb))(*cb)
        eng.lib.RunShader(name.encode(), sa, ns, ua, nu, th, ctypes.cast(cba, ctypes.c_void_p), 4 * len(cb))
    else:
        eng.lib.RunShader(name.encode(), sa, ns, ua, nu, th, None, 0)


def new(eng, n):
    h = eng.lib.CreateBuffer(None, n)
    assert h, eng.last_error()
    return h


@pytest.fixture(params=["cached", "streaming"])
def policy(request, eng):
    """Run a test with the default cache policy and again with every pass
    forced onto the nontemporal (streaming) kernel forms, which by default
    only passes over 256 MiB take."""
    if request.param == "cached":
        yield request.param
        return
    prev = eng.lib.SetStreamingThreshold(0.0)
    try:
        yield request.param
    finally:
        eng.lib.SetStreamingThreshold(prev)


# ----------------------------------------------------------------- buffers
def test_buffer_roundtrip_update_clear(eng):
    for n in (1, 7, 256, 257, 100003, 5_000_000):
        a = rng(n).standard_normal(n).astype(np.float32)
        h = upload(eng, a)
        assert np.array_equal(download(eng, h, (n,)), a)
        b = rng(n + 1).standard_normal(n).astype(np.float32)
        eng.lib.UpdateBuffer(h, b.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        assert np.array_equal(download(eng, h, (n,)), b)
        eng.lib.ClearBuffer(h)
        assert not download(eng, h, (n,)).any()
        release(eng, h)


def test_refcount_pool_and_errors(eng):
    lib = eng.lib
    assert lib.CreateBuffer(None, 0) is None          # zero-size: NULL + error
    assert "zero-size" in eng.last_error()
    h = new(eng, 1000)
    lib.AddRefBuffer(h)
    lib.ReleaseBuffer(h)                               # still referenced
    lib.ClearBuffer(h)
    lib.ReleaseBuffer(h)                               # back to the pool
    lib.ClearLastError()
    lib.ReleaseBuffer(h)                               # double release: rejected, no crash
    assert "not live" in eng.last_error()
    lib.ResetPoolStats()
    h2 = new(eng, 1000)                                # pool hit (same size)
    hits, misses = eng.get_pool_stats()
    assert hits >= 1
    arr = (ctypes.c_void_p * 2)(h2, None)
    lib.ReleaseBufferBatch(arr, 2)                     # NULL entries skipped
    sizes = (ctypes.c_uint * 2)(12345, 777)
    lib.WarmPool(sizes, 2, 3)
    assert lib.GetPoolMemory() >= (12345 + 777) * 4 * 3
    lib.DrainPool()
    assert lib.GetPoolMemory() == 0


def test_gpu_info(eng):
    info = eng.GPUInfo()
    eng.lib.GetGPUInfo(ctypes.byref(info))
    assert info.vendorId == 0x1002 and info.isIntegrated == 0
    assert info.dedicatedVRAM > (64 << 30)
    assert b"gfx950" in info.description


def test_fused_calls_reject_bad_geometry(eng):
    """The fused entry points return NULL, and leave the reason in
    GetLastErrorString, for buffers smaller than their geometry, invalid
    geometry, and sizes past 31-bit indexing (the filters' included), so no
    kernel runs over memory the buffers do not hold."""
    lib = eng.lib
    small = new(eng, 16)
    w, b = new(eng, 8 * 4 * 3 * 3), new(eng, 8)

    def rejected(h, what):
        assert not h
        err = eng.last_error()
        assert what in err, err
        lib.ClearLastError()

    rejected(lib.ConvForwardFused(small, w, b, 2, 4, 8, 8, 8, 3, 3, 1, 1, 0, None), "smaller")
    rejected(lib.ConvForwardFused(small, w, b, 1, 4, 2, 2, 8, 5, 5, 1, 0, 0, None), "invalid geometry")
    # 65536 x 65536 1x1 filters on a 1x1 image: activations fit, the filters do not.
    rejected(lib.ConvForwardFused(small, small, small, 1, 65536, 1, 1, 65536, 1, 1, 1, 0, 0, None),
             "too large")
    pdf, pdb, pdx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
    lib.ConvBackwardFused(small, None, small, w, None, 2, 4, 8, 8, 8, 3, 3, 1, 1, 0, 1, 1, 1,
                          ctypes.byref(pdf), ctypes.byref(pdb), ctypes.byref(pdx))
    assert not (pdf.value or pdb.value or pdx.value)
    rejected(None, "smaller")
    rejected(lib.MatMulAlloc(small, small, 64, 64, 64, 0), "smaller")
    pidx = ctypes.c_void_p()
    rejected(lib.MaxPoolForwardFused(small, 2, 4, 8, 8, 2, 2, ctypes.byref(pidx)), "does not match")
    assert not pidx.value
    # MaxPoolBackwardFused consumes its index handle, error or not.
    rejected(lib.MaxPoolBackwardFused(small, new(eng, 16), 65536, 65536, 1, 1, 16), "too large")
    rejected(lib.MaxPoolBackwardFused(small, new(eng, 16), 2, 4, 4, 4, 64), "smaller")
    release(eng, small, w, b)


def test_unknown_shader_is_noop_with_error(eng):
    h = upload(eng, np.ones(4, np.float32))
    eng.lib.ClearLastError()
    run(eng, "gelu", [h], [h], 4)
    assert "unknown kernel" in eng.last_error()
    assert np.array_equal(download(eng, h, (4,)), np.ones(4, np.float32))
    release(eng, h)


# ------------------------------------------------------------ elementwise
UNARY = [
    ("relu", lambda x: K.relu(x), False),
    ("relu6", lambda x: K.relu6(x), True),
    ("sigmoid", lambda x: K.sigmoid(x), True),
]
BINARY = [
    ("relu_grad", K.relu_grad),
    ("relu6_grad", K.relu6_grad),
    ("sigmoid_grad", K.sigmoid_grad),
]


@pytest.mark.parametrize("n", [1, 5, 1024, 1000003] +
                         [int(v) for v in np.random.default_rng(919).integers(2, 300000, 4)])
def test_activations(eng, n, policy):
    r = rng(n)
    x = (4 * r.standard_normal(n)).astype(np.float32)
    x[: min(n, 3)] = [0.0, 6.0, -0.0][: min(n, 3)]
    g = r.standard_normal(n).astype(np.float32)
    hx, hg = upload(eng, x), upload(eng, g)
    for name, fn, has_cb in UNARY:
        ho = new(eng, n)
        run(eng, name, [hx], [ho], *([n] if has_cb else []))
        assert rel_err(download(eng, ho, (n,)), fn(x)) <= 1e-6, name
        release(eng, ho)
    for name, fn in BINARY:
        ho = new(eng, n)
        run(eng, name, [hg, hx], [ho], n)
        assert rel_err(download(eng, ho, (n,)), fn(g, x)) <= 1e-6, name
        release(eng, ho)
    for alpha in (0.1, 0.01):
        ho = new(eng, n)
        run(eng, "leaky_relu", [hx], [ho], n, fbits(alpha))
        assert rel_err(download(eng, ho, (n,)), K.leaky_relu(x, alpha)) <= 1e-6
        run(eng, "leaky_relu_grad", [hg, hx], [ho], n, fbits(alpha))
        assert rel_err(download(eng, ho, (n,)), K.leaky_relu_grad(g, x, alpha)) <= 1e-6
        release(eng, ho)
    ho = new(eng, n)
    run(eng, "add", [hx, hg], [ho], n, 1)
    assert rel_err(download(eng, ho, (n,)), x.astype(np.float64) + g) <= 1e-6
    run(eng, "scale_add", [hx, hg], [ho], n, fbits(1.5), fbits(-0.5))
    assert rel_err(download(eng, ho, (n,)), 1.5 * x.astype(np.float64) - 0.5 * g) <= 1e-6
    acc = upload(eng, x)
    run(eng, "grad_accum", [hg], [acc], n)
    assert rel_err(download(eng, acc, (n,)), K.grad_accum(x, g)) <= 1e-6
    release(eng, hx, hg, ho, acc)


def test_out_of_bounds_reads_zero_writes_dropped(eng):
    """D3D11 structured-buffer rules: count larger than the buffers reads 0 and
    drops writes beyond the output (nn_relu.hlsl relies on it)."""
    g = np.arange(1, 11, dtype=np.float32)
    x = np.ones(6, np.float32)
    hg, hx = upload(eng, g), upload(eng, x)
    ho = upload(eng, np.full(8, 7.0, np.float32))
    run(eng, "relu_grad", [hg, hx], [ho], 100)
    out = download(eng, ho, (8,))
    assert np.array_equal(out, np.array([1, 2, 3, 4, 5, 6, 0, 0], np.float32))
    run(eng, "relu", [hg], [ho])            # no constants: bounded by the output
    assert np.array_equal(download(eng, ho, (8,)), g[:8])
    release(eng, hg, hx, ho)


@pytest.mark.parametrize("M,N", [(1, 1), (128, 4096), (7, 13), (64, 10)])
def test_bias_ops(eng, M, N):
    r = rng(M * N)
    A = r.standard_normal((M, N)).astype(np.float32)
    b = r.standard_normal(N).astype(np.float32)
    hA, hb, ho = upload(eng, A), upload(eng, b), new(eng, M * N)
    run(eng, "add_bias", [hA, hb], [ho], M, N)
    assert rel_err(download(eng, ho, (M, N)), K.add_bias(A, b)) <= 1e-6
    run(eng, "bias_relu", [hA, hb], [ho], M, N)
    assert rel_err(download(eng, ho, (M, N)), K.bias_relu(A, b)) <= 1e-6
    hg = new(eng, N)
    run(eng, "bias_grad", [hA], [hg], M, N, N, 1)          # linear layout
    assert rel_err(download(eng, hg, (N,)), K.bias_grad(A, M, N, N, 1)) <= TOL
    hg2 = new(eng, M)
    run(eng, "bias_grad", [hA], [hg2], N, M, 1, N)         # conv layout (rows contiguous)
    assert rel_err(download(eng, hg2, (M,)), K.bias_grad(A, N, M, 1, N)) <= TOL
    release(eng, hA, hb, ho, hg, hg2)


# ----------------------------------------------------------------- maxpool
POOL_CASES = [(2, 3, 8, 8, 2, 2), (2, 4, 55, 55, 3, 2), (1, 2, 27, 27, 3, 2), (3, 5, 13, 11, 3, 2),
              (2, 3, 9, 9, 3, 1), (1, 6, 24, 24, 2, 2), (2, 2, 7, 10, 2, 3), (2, 3, 9, 7, 2, 2),
              (1, 2, 256, 200, 2, 2), (1, 2, 121, 301, 3, 2), (1, 1, 9, 8199, 3, 2),
              # 3x3 s2 around the paired-window path's limits: one window column
              # (scalar path), two columns, and an even width
              (2, 3, 5, 4, 3, 2), (2, 3, 6, 5, 3, 2), (2, 3, 10, 56, 3, 2),
              # 2x2 s2: the two-window quad path (even output width) and an odd one
              (2, 16, 64, 64, 2, 2), (1, 2, 12, 10, 2, 2)]


@pytest.mark.parametrize("B,C,H,W,k,s", POOL_CASES)
def test_maxpool_fused(eng, B, C, H, W, k, s):
    r = rng(B * C * H * W + k)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    x.flat[::17] = 0.5              # ties: first candidate in scan order wins
    x.flat[5::97] = np.nan          # NaN is never selected (strict '>')
    x.flat[0] = -np.inf
    hx = upload(eng, x)
    pidx = ctypes.c_void_p()
    ho = eng.lib.MaxPoolForwardFused(hx, B, C, H, W, k, s, ctypes.byref(pidx))
    assert ho, eng.last_error()
    OH, OW = (H - k) // s + 1, (W - k) // s + 1
    out = download(eng, ho, (B, C, OH, OW))
    idx = download(eng, pidx.value, (B, C, OH, OW)).view(np.uint32)
    ref_out, ref_idx = K.maxpool_forward(x, k, s)
    assert np.array_equal(idx, ref_idx)                      # bit-exact routing
    assert np.array_equal(out, ref_out.astype(np.float32))
    dz = r.standard_normal((B, C, OH, OW)).astype(np.float32)
    hdz = upload(eng, dz)
    hdx = eng.lib.MaxPoolBackwardFused(hdz, pidx.value, B, C, OH, OW, x.size)
    assert hdx, eng.last_error()
    dx = download(eng, hdx, x.shape)
    ref_dx = K.maxpool_backward(dz, ref_idx, x.size).reshape(x.shape)
    if k <= s:
        assert np.array_equal(dx, ref_dx.astype(np.float32))  # disjoint windows: exact
    else:
        assert rel_err(dx, ref_dx) <= 1e-6
    release(eng, hx, ho, hdz, hdx)


def test_maxpool_raw_shaders(eng):
    B, C, H, W, k, s = 2, 3, 8, 8, 2, 2
    x = rng(3).standard_normal((B, C, H, W)).astype(np.float32)
    OH = OW = 4
    hx, ho, hi = upload(eng, x), new(eng, B * C * 16), new(eng, B * C * 16)
    run(eng, "maxpool_forward", [hx], [ho, hi], B, C, H, W, k, s, OH, OW)
    ref_out, ref_idx = K.maxpool_forward(x, k, s)
    assert np.array_equal(download(eng, hi, (B, C, OH, OW)).view(np.uint32), ref_idx)
    dz = rng(4).standard_normal((B, C, OH, OW)).astype(np.float32)
    hdz, hdx = upload(eng, dz), new(eng, x.size)
    eng.lib.ClearBuffer(hdx)
    run(eng, "maxpool_backward", [hdz, hi], [hdx], B, C, OH, OW)
    assert np.array_equal(download(eng, hdx, x.shape), K.maxpool_backward(dz, ref_idx, x.size).reshape(x.shape).astype(np.float32))
    release(eng, hx, ho, hi, hdz, hdx)


@pytest.mark.parametrize("planes,outPer,inPer", [(6, 729, 3025), (3, 700, 40), (2, 300, 20000)],
                         ids=["lds_pool1", "lds_dense_dups", "per_thread_large_plane"])
def test_maxpool_backward_arbitrary_indices(eng, planes, outPer, inPer):
    """MaxPoolBackwardFused on caller indices that no pooling window could
    make: many outputs per input (duplicates inside one 256-output round of
    the LDS kernel), indices in another plane and the 0xFFFFFFFF marker.  Each
    input must add its plane's contributions one by one in output order, so
    the result equals a float32 np.add.at in that order bit for bit (planes
    up to 14336 inputs take the LDS kernel, larger ones the per-thread one)."""
    r = rng(planes * outPer + inPer)
    dz = r.standard_normal(planes * outPer).astype(np.float32)
    local = r.integers(0, min(inPer, 97), planes * outPer)          # heavy duplication
    idx = (np.repeat(np.arange(planes), outPer) * inPer + local).astype(np.uint32)
    idx[::17] = 0xFFFFFFFF                                           # no argmax
    idx[5::23] = (idx[5::23] + inPer) % (planes * inPer)             # another plane: dropped
    ref = np.zeros(planes * inPer, np.float32)
    keep = (idx != 0xFFFFFFFF) & (idx // inPer == np.repeat(np.arange(planes), outPer))
    np.add.at(ref, idx[keep].astype(np.int64), dz[keep])
    hdz = upload(eng, dz)
    for _ in range(2):
        hi = upload(eng, idx.view(np.float32))
        eng.lib.ClearLastError()
        hdx = eng.lib.MaxPoolBackwardFused(hdz, hi, planes, 1, outPer, 1, planes * inPer)
        assert hdx, eng.last_error()
        assert np.array_equal(download(eng, hdx, ref.shape), ref)
        release(eng, hdx)
    release(eng, hdz)


@pytest.mark.parametrize("B,C,H,W,k,s", [(2, 4, 55, 55, 3, 2), (2, 3, 8, 8, 2, 2), (1, 2, 9, 9, 3, 1)])
def test_maxpool_backward_untagged_indices(eng, B, C, H, W, k, s):
    """MaxPoolBackwardFused on indices that carry no pooling geometry (here a
    copy the caller uploaded): the per-plane fallback sums every window in
    (oh, ow) order, the gather kernels' order, so it matches the tagged path
    bit for bit and the oracle's routing; no float atomics, so it repeats
    exactly.  Indices from RunShader("maxpool_forward") carry the geometry."""
    r = rng(B * C * H * W + 11)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    x.flat[::13] = 0.25             # ties
    OH, OW = (H - k) // s + 1, (W - k) // s + 1
    ref_out, ref_idx = K.maxpool_forward(x, k, s)
    dz = r.standard_normal((B, C, OH, OW)).astype(np.float32)
    hx, hdz = upload(eng, x), upload(eng, dz)
    outs = []
    for kind in ("fused", "runshader", "uploaded", "uploaded"):
        if kind == "fused":
            pidx = ctypes.c_void_p()
            ho = eng.lib.MaxPoolForwardFused(hx, B, C, H, W, k, s, ctypes.byref(pidx))
            hi = pidx.value
        elif kind == "runshader":
            ho, hi = new(eng, ref_idx.size), new(eng, ref_idx.size)
            run(eng, "maxpool_forward", [hx], [ho, hi], B, C, H, W, k, s, OH, OW)
        else:
            ho, hi = None, upload(eng, ref_idx.view(np.float32))
        eng.lib.ClearLastError()
        hdx = eng.lib.MaxPoolBackwardFused(hdz, hi, B, C, OH, OW, x.size)   # consumes hi
        assert hdx, eng.last_error()
        outs.append(download(eng, hdx, x.shape))
        release(eng, ho, hdx)
    ref_dx = K.maxpool_backward(dz, ref_idx, x.size).reshape(x.shape)
    for o in outs:
        assert np.array_equal(o, outs[0])
    assert rel_err(outs[0], ref_dx) <= 1e-6
    if k <= s:
        assert np.array_equal(outs[0], ref_dx.astype(np.float32))
    # an index outside its own (b, c) plane cannot come from a pooling window
    bad = ref_idx.copy().reshape(-1)
    bad[0] = x.size - 1
    hi = upload(eng, bad.view(np.float32))
    hdx = eng.lib.MaxPoolBackwardFused(hdz, hi, B, C, OH, OW, x.size)
    assert hdx, eng.last_error()
    got = download(eng, hdx, x.shape).reshape(-1)
    keep = np.ones(bad.size, bool)
    keep[0] = False
    exp = K.maxpool_backward(dz.reshape(-1)[keep], bad[keep], x.size)
    assert rel_err(got, exp) <= 1e-6
    release(eng, hdx)
    # no geometry and an input size that is not a whole number of planes
    hi = upload(eng, ref_idx.view(np.float32))
    assert not eng.lib.MaxPoolBackwardFused(hdz, hi, B, C, OH, OW, x.size + 1)
    assert "not a multiple" in eng.last_error()
    release(eng, hx, hdz)


# ---------------------------------------------------------------- batchnorm
@pytest.mark.parametrize("N,C,H,W", [(2, 3, 5, 5), (8, 16, 32, 32), (4, 96, 28, 28), (64, 6, 12, 12), (1, 1, 1, 7),
                                     (16, 4, 64, 64)])
def test_batchnorm(eng, N, C, H, W, policy):
    r = rng(N * C * H * W)
    x = (r.standard_normal((N, C, H, W)) * 2 + 0.5).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(C)).astype(np.float32)
    beta = (0.1 * r.standard_normal(C)).astype(np.float32)
    rm = (0.1 * r.standard_normal(C)).astype(np.float32)
    rv = (1 + 0.1 * r.random(C)).astype(np.float32)
    dy = r.standard_normal(x.shape).astype(np.float32)
    eps, mom = 1e-5, 0.1
    S = H * W
    hx, hg, hb, hrm, hrv, hdy = (upload(eng, a) for a in (x, gamma, beta, rm, rv, dy))
    hmu, hvar = new(eng, C), new(eng, C)
    run(eng, "batchnorm_mean_var", [hx], [hmu, hvar, hrm, hrv], N, C, S, 1, fbits(mom))
    mu_r, var_r, rm_r, rv_r = K.batchnorm_mean_var(x, rm, rv, mom, True)
    mu, var = download(eng, hmu, (C,)), download(eng, hvar, (C,))
    assert rel_err(mu, mu_r) <= 1e-5 and rel_err(var, var_r) <= 1e-5
    assert rel_err(download(eng, hrm, (C,)), rm_r) <= 1e-5
    assert rel_err(download(eng, hrv, (C,)), rv_r) <= 1e-5
    hy = new(eng, x.size)
    run(eng, "batchnorm_forward", [hx, hmu, hvar, hg, hb], [hy], N, C, S, fbits(eps))
    assert rel_err(download(eng, hy, x.shape), K.batchnorm_forward(x, mu, var, gamma, beta, eps)) <= 1e-5
    hdg, hdb = new(eng, C), new(eng, C)
    run(eng, "batchnorm_backward_reduce", [hx, hdy, hmu, hvar], [hdg, hdb], N, C, S, fbits(eps))
    dg_r, db_r = K.batchnorm_backward_reduce(x, dy, mu, var, eps)
    dg, db = download(eng, hdg, (C,)), download(eng, hdb, (C,))
    assert rel_err(dg, dg_r) <= TOL and rel_err(db, db_r) <= TOL
    hdx = new(eng, x.size)
    run(eng, "batchnorm_backward_dx", [hx, hdy, hmu, hvar, hg, hdg, hdb], [hdx], N, C, S, fbits(eps))
    dx_r = K.batchnorm_backward_dx(x, dy, mu, var, gamma, dg, db, eps)
    assert rel_err(download(eng, hdx, x.shape), dx_r) <= TOL
    release(eng, hx, hg, hb, hrm, hrv, hdy, hmu, hvar, hy, hdg, hdb, hdx)


# --------------------------------------------------- pooling / resampling
@pytest.mark.parametrize("B,C,H,W", [(2, 3, 7, 7), (8, 64, 8, 8), (1, 1, 1, 1)] +
                         [tuple(int(v) for v in np.random.default_rng(717 + i).integers([1, 1, 1, 1], [9, 70, 40, 40]))
                          for i in range(6)])
def test_global_avg_pool(eng, B, C, H, W, policy):
    x = rng(B + C).standard_normal((B, C, H, W)).astype(np.float32)
    g = rng(7).standard_normal((B, C)).astype(np.float32)
    hx, ho, hg, hdx = upload(eng, x), new(eng, B * C), upload(eng, g), new(eng, x.size)
    run(eng, "global_avg_pool", [hx], [ho], B, C, H * W)
    assert rel_err(download(eng, ho, (B, C)), K.global_avg_pool(x)) <= 1e-6
    run(eng, "global_avg_pool_backward", [hg], [hdx], B, C, H * W)
    assert rel_err(download(eng, hdx, x.shape), K.global_avg_pool_backward(g, x.shape)) <= 1e-6
    release(eng, hx, ho, hg, hdx)


@pytest.mark.parametrize("B,C,H,W,sH,sW", [(2, 3, 4, 5, 2, 2), (1, 16, 32, 32, 2, 2), (2, 2, 3, 3, 3, 2),
                                           (2, 4, 6, 2, 2, 2), (1, 8, 1, 4, 2, 2), (3, 5, 7, 10, 2, 2)] +
                         [tuple(int(v) for v in np.random.default_rng(818 + i).integers([1, 1, 1, 1, 1, 1],
                                                                                        [5, 20, 40, 40, 4, 4]))
                          for i in range(6)])
def test_upsample(eng, B, C, H, W, sH, sW, policy):
    x = rng(H * W).standard_normal((B, C, H, W)).astype(np.float32)
    OH, OW = H * sH, W * sW
    dy = rng(5).standard_normal((B, C, OH, OW)).astype(np.float32)
    hx, hy, hdy, hdx = upload(eng, x), new(eng, B * C * OH * OW), upload(eng, dy), new(eng, x.size)
    run(eng, "upsample", [hx], [hy], B, C, H, W, OH, OW, sH, sW)
    assert np.array_equal(download(eng, hy, dy.shape), K.upsample(x, sH, sW).astype(np.float32))
    run(eng, "upsample_backward", [hdy], [hdx], B, C, H, W, OH, OW, sH, sW)
    assert rel_err(download(eng, hdx, x.shape), K.upsample_backward(dy, x.shape, sH, sW)) <= 1e-6
    release(eng, hx, hy, hdy, hdx)


@pytest.mark.parametrize("H,W", [(4, 5), (3, 5)])   # plane sizes 20 (quad path) and 15
def test_concat_slice(eng, H, W, policy):
    B, S = 2, H * W
    a = rng(1).standard_normal((B, 3, H, W)).astype(np.float32)
    b = rng(2).standard_normal((B, 5, H, W)).astype(np.float32)
    ha, hb, ho = upload(eng, a), upload(eng, b), new(eng, B * 8 * S)
    run(eng, "concat_insert", [ha], [ho], B, 3, S, 8, 0)
    run(eng, "concat_insert", [hb], [ho], B, 5, S, 8, 3)
    cat = download(eng, ho, (B, 8, H, W))
    assert np.array_equal(cat, K.concat([a, b]).astype(np.float32))
    hs = new(eng, B * 5 * S)
    run(eng, "slice", [ho], [hs], B, 5, S, 8, 3)
    assert np.array_equal(download(eng, hs, b.shape), b)
    release(eng, ha, hb, ho, hs)


# ---------------------------------------------------------------- depthwise
DW_CASES = [
    (2, 8, 9, 9, 3, 1, 1), (2, 6, 10, 12, 3, 2, 1), (1, 4, 7, 7, 5, 1, 2), (4, 96, 28, 28, 3, 2, 1),
    # band kernels: several bands per plane, K 5 stride 2, pad 0, one-row bands on a wide plane
    (2, 16, 56, 56, 3, 1, 1), (2, 16, 112, 112, 3, 2, 1), (2, 5, 11, 13, 5, 2, 2), (2, 3, 8, 9, 3, 1, 0),
    (1, 2, 3, 1100, 3, 1, 1),
    # quad windows (row widths multiples of 4), shifted window origins, mixed dword / quad
    (2, 4, 32, 32, 5, 1, 2), (2, 4, 40, 40, 5, 2, 2), (2, 4, 31, 33, 3, 2, 0), (2, 4, 18, 18, 3, 1, 0),
    (2, 3, 25, 25, 5, 2, 1), (1, 2, 200, 64, 3, 1, 1),
    # generic kernels: 2x2 taps, stride 3
    (2, 4, 8, 8, 2, 2, 0), (1, 4, 10, 10, 3, 3, 1),
]


@pytest.mark.parametrize("B,C,H,W,k,s,p", DW_CASES)
def test_depthwise(eng, B, C, H, W, k, s, p, policy):
    r = rng(B * C * H + k + s)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    f = r.standard_normal((C, 1, k, k)).astype(np.float32)
    b = r.standard_normal(C).astype(np.float32)
    OH, OW = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    dy = r.standard_normal((B, C, OH, OW)).astype(np.float32)
    hx, hf, hb, hdy = upload(eng, x), upload(eng, f), upload(eng, b), upload(eng, dy)
    hy, hdx, hdf, hdb = new(eng, dy.size), new(eng, x.size), new(eng, f.size), new(eng, C)
    cb = (B, C, H, W, k, k, s, p, OH)
    run(eng, "depthwise_conv_forward", [hx, hf, hb], [hy], *cb)
    assert rel_err(download(eng, hy, dy.shape), K.depthwise_forward(x, f, b, s, p)) <= 1e-5
    run(eng, "depthwise_conv_backward_input", [hdy, hf], [hdx], *cb)
    assert rel_err(download(eng, hdx, x.shape), K.depthwise_backward_input(dy, f, x.shape, s, p)) <= TOL
    run(eng, "depthwise_conv_backward_filter", [hdy, hx], [hdf, hdb], *cb)
    df_r, db_r = K.depthwise_backward_filter(dy, x, k, k, s, p)
    assert rel_err(download(eng, hdf, f.shape), df_r) <= TOL
    assert rel_err(download(eng, hdb, (C,)), db_r) <= TOL
    release(eng, hx, hf, hb, hdy, hy, hdx, hdf, hdb)


def _random_dw_cases(n, seed):
    """Seeded depthwise geometries: K in {3, 5}, stride 1 or 2, every padding
    below K, odd and even plane sizes from K to 69, 1-39 channels."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k, s = int(r.choice([3, 5])), int(r.choice([1, 2]))
        p = int(r.integers(0, k))
        H, W = int(r.integers(k, 70)), int(r.integers(k, 70))
        out.append((int(r.integers(1, 4)), int(r.integers(1, 40)), H, W, k, s, p))
    return out


DW_RANDOM = _random_dw_cases(24, 2718)


@pytest.mark.parametrize("case", DW_RANDOM, ids=["x".join(map(str, c)) for c in DW_RANDOM])
def test_depthwise_random_geometries(eng, case):
    """Depthwise forward, dX, dW and db on seeded random geometries (band and
    generic kernels, quad and dword windows) against the float64 oracle."""
    test_depthwise(eng, *case, policy="cached")


def _random_pool_cases(n, seed):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k, s = int(r.choice([2, 3])), int(r.choice([1, 2, 3]))
        out.append((int(r.integers(1, 4)), int(r.integers(1, 20)), int(r.integers(k, 60)),
                    int(r.integers(k, 60)), k, s))
    return out


POOL_RANDOM = _random_pool_cases(16, 1618)


@pytest.mark.parametrize("case", POOL_RANDOM, ids=["x".join(map(str, c)) for c in POOL_RANDOM])
def test_maxpool_random_geometries(eng, case):
    """Fused max-pool forward (values, indices) and backward routing on seeded
    random geometries, overlapping and gapped windows included."""
    test_maxpool_fused(eng, *case)


BN_RANDOM = [tuple(int(v) for v in np.random.default_rng(1414 + i).integers([1, 1, 1, 1], [9, 48, 40, 40]))
             for i in range(12)]


@pytest.mark.parametrize("case", BN_RANDOM, ids=["x".join(map(str, c)) for c in BN_RANDOM])
def test_batchnorm_random_shapes(eng, case):
    """BatchNorm statistics, forward and backward on seeded random shapes."""
    test_batchnorm(eng, *case, policy="cached")


# ------------------------------------- MobileNetV2 b64 @112^2 at full size
@pytest.mark.parametrize("B,C,H,W,s", [(64, 96, 112, 112, 2), (64, 144, 56, 56, 1), (64, 192, 28, 28, 1)])
def test_mobilenet_b64_block_full_size_sampled(eng, B, C, H, W, s):
    """The expanded tensors of the MobileNetV2 stack's blocks at the timed
    size (b64 @112^2): BN statistics and forward, ReLU6, depthwise 3x3
    forward and backward, ReLU6 gradient and BN backward over the whole
    tensor, with the piece counts, band plans and streaming forms this size
    selects (passes over 256 MiB).  Channels are independent in all of them,
    so each sampled channel is checked against the float64 oracle over the
    full batch exactly.  Every stage takes the device's previous output as
    its input, as the training step does."""
    r = rng(C * H)
    x = (r.standard_normal((B, C, H, W)) * 2 + 0.5).astype(np.float32)
    gamma = (1 + 0.1 * r.standard_normal(C)).astype(np.float32)
    beta = (0.1 * r.standard_normal(C)).astype(np.float32)
    f = (r.standard_normal((C, 1, 3, 3)) / 3).astype(np.float32)
    fb = (0.1 * r.standard_normal(C)).astype(np.float32)
    OH, OW = (H - 1) // s + 1, (W - 1) // s + 1
    dz = r.standard_normal((B, C, OH, OW)).astype(np.float32)
    cs = [0, C // 2 + 1, C - 1]
    n, eps, mom = x.size, 1e-5, 0.1
    shp = (B, C, H, W)
    hx, hg, hb, hf, hfb, hdz = (upload(eng, a) for a in (x, gamma, beta, f, fb, dz))
    hrm, hrv = upload(eng, np.zeros(C, np.float32)), upload(eng, np.ones(C, np.float32))
    hmu, hvar, hy, ha = new(eng, C), new(eng, C), new(eng, n), new(eng, n)
    hz, hda, hdf, hdfb = new(eng, dz.size), new(eng, n), new(eng, f.size), new(eng, C)
    hdy, hdg, hdbe, hdx = new(eng, n), new(eng, C), new(eng, C), new(eng, n)
    xs = x[:, cs]

    run(eng, "batchnorm_mean_var", [hx], [hmu, hvar, hrm, hrv], B, C, H * W, 1, fbits(mom))
    mu, var = download(eng, hmu, (C,)), download(eng, hvar, (C,))
    mu_r, var_r, _, _ = K.batchnorm_mean_var(xs, np.zeros(3), np.ones(3), mom, True)
    assert rel_err(mu[cs], mu_r) <= 1e-5 and rel_err(var[cs], var_r) <= 1e-5
    run(eng, "batchnorm_forward", [hx, hmu, hvar, hg, hb], [hy], B, C, H * W, fbits(eps))
    y = download(eng, hy, shp)[:, cs]
    assert rel_err(y, K.batchnorm_forward(xs, mu[cs], var[cs], gamma[cs], beta[cs], eps)) <= 1e-5
    run(eng, "relu6", [hy], [ha], n)
    a = download(eng, ha, shp)[:, cs]
    assert rel_err(a, K.relu6(y)) <= 1e-6
    cb = (B, C, H, W, 3, 3, s, 1, OH)
    run(eng, "depthwise_conv_forward", [ha, hf, hfb], [hz], *cb)
    z = download(eng, hz, dz.shape)[:, cs]
    assert rel_err(z, K.depthwise_forward(a, f[cs], fb[cs], s, 1)) <= 1e-5
    run(eng, "depthwise_conv_backward_input", [hdz, hf], [hda], *cb)
    da = download(eng, hda, shp)[:, cs]
    assert rel_err(da, K.depthwise_backward_input(dz[:, cs], f[cs], a.shape, s, 1)) <= TOL
    run(eng, "depthwise_conv_backward_filter", [hdz, ha], [hdf, hdfb], *cb)
    df_r, dfb_r = K.depthwise_backward_filter(dz[:, cs], a, 3, 3, s, 1)
    assert rel_err(download(eng, hdf, f.shape)[cs], df_r) <= TOL
    assert rel_err(download(eng, hdfb, (C,))[cs], dfb_r) <= TOL
    run(eng, "relu6_grad", [hda, hy], [hdy], n)
    dy = download(eng, hdy, shp)[:, cs]
    assert rel_err(dy, K.relu6_grad(da, y)) <= 1e-6
    run(eng, "batchnorm_backward_reduce", [hx, hdy, hmu, hvar], [hdg, hdbe], B, C, H * W, fbits(eps))
    dg, dbe = download(eng, hdg, (C,)), download(eng, hdbe, (C,))
    dg_r, dbe_r = K.batchnorm_backward_reduce(xs, dy, mu[cs], var[cs], eps)
    assert rel_err(dg[cs], dg_r) <= TOL and rel_err(dbe[cs], dbe_r) <= TOL
    run(eng, "batchnorm_backward_dx", [hx, hdy, hmu, hvar, hg, hdg, hdbe], [hdx], B, C, H * W, fbits(eps))
    dx_r = K.batchnorm_backward_dx(xs, dy, mu[cs], var[cs], gamma[cs], dg[cs], dbe[cs], eps)
    assert rel_err(download(eng, hdx, shp)[:, cs], dx_r) <= TOL
    release(eng, hx, hg, hb, hf, hfb, hdz, hrm, hrv, hmu, hvar, hy, ha, hz, hda, hdf, hdfb, hdy, hdg,
            hdbe, hdx)


# ------------------------------------------------------------ loss / metrics
SOFTMAX_RANDOM = [tuple(int(v) for v in np.random.default_rng(515 + i).integers([1, 2], [260, 3000]))
                  for i in range(8)]   # seeded: class counts past the 1024-class register rows too


@pytest.mark.parametrize("B,Kc", [(1, 2), (64, 10), (128, 1000), (300, 7)] + SOFTMAX_RANDOM)
def test_softmax_ce(eng, B, Kc):
    r = rng(B * Kc)
    z = (3 * r.standard_normal((B, Kc))).astype(np.float32)
    lab = r.integers(0, Kc, B).astype(np.float32)
    hz, hl = upload(eng, z), upload(eng, lab)
    hp, hloss, hg = new(eng, B * Kc), new(eng, 1), new(eng, B * Kc)
    run(eng, "softmax", [hz], [hp], B, Kc)
    p = download(eng, hp, (B, Kc))
    assert rel_err(p, K.softmax(z)) <= 1e-5
    run(eng, "loss", [hz, hl], [hloss], B, Kc)
    assert abs(download(eng, hloss, (1,))[0] - K.ce_loss(z, lab)) <= 1e-5 * max(1, K.ce_loss(z, lab))
    run(eng, "softmax_ce_grad", [hp, hl], [hg], B, Kc)
    assert rel_err(download(eng, hg, (B, Kc)), K.softmax_ce_grad(p, lab)) <= 1e-5
    hc = new(eng, 1)
    eng.lib.ClearBuffer(hc)
    z[0, :] = 1.0  # all-equal row: first column wins
    hz2 = upload(eng, z)
    run(eng, "argmax_correct", [hz2, hl], [hc], B, Kc)
    run(eng, "argmax_correct", [hz2, hl], [hc], B, Kc)
    cnt = download(eng, hc, (1,)).view(np.uint32)[0]
    assert cnt == 2 * K.argmax_correct(z, lab)                 # bit-exact count
    acc = upload(eng, np.array([1.5], np.float32))
    run(eng, "accumulate_scalar", [hloss], [acc])
    assert abs(download(eng, acc, (1,))[0] - (1.5 + download(eng, hloss, (1,))[0])) < 1e-6
    release(eng, hz, hl, hp, hloss, hg, hc, hz2, acc)


@pytest.mark.parametrize("B,C,H,W", [(2, 1, 16, 16), (8, 1, 64, 64), (3, 2, 5, 7), (8, 1, 256, 256)] +
                         [tuple(int(v) for v in np.random.default_rng(616 + i).integers([1, 1, 1, 1], [9, 3, 90, 90]))
                          for i in range(6)])
def test_dice(eng, B, C, H, W):
    r = rng(B * H)
    p = r.random((B, C, H, W)).astype(np.float32)
    t = (r.random((B, C, H, W)) < 0.3).astype(np.float32)
    size = C * H * W
    hp, ht = upload(eng, p), upload(eng, t)
    hl, hs, hg = new(eng, B), new(eng, 3 * B), new(eng, p.size)
    run(eng, "dice_loss", [hp, ht], [hl], B, size)
    assert rel_err(download(eng, hl, (B,)), K.dice_loss(p, t)) <= 1e-5
    run(eng, "dice_loss_sums", [hp, ht], [hs], B, size)
    assert rel_err(download(eng, hs, (B, 3)), K.dice_sums(p, t)) <= 1e-5
    run(eng, "dice_loss_grad", [hp, ht, hs], [hg], B, size)
    assert rel_err(download(eng, hg, p.shape), K.dice_loss_grad(p, t)) <= TOL
    release(eng, hp, ht, hl, hs, hg)


# ---------------------------------------------------------------- optimisers
def _param_set(seed, sizes):
    r = rng(seed)
    return ([r.standard_normal(n).astype(np.float32) for n in sizes],
            [(2 * r.standard_normal(n)).astype(np.float32) for n in sizes])


SIZES = [1, 3, 4, 5, 4095, 4096, 4097, 100000, 9216 * 40]


def _arrays(hs):
    return (ctypes.c_void_p * len(hs))(*hs)


def test_sgd_batch(eng, policy):
    ws, gs = _param_set(1, SIZES)
    hw, hg = [upload(eng, w) for w in ws], [upload(eng, g) for g in gs]
    pa, ga = _arrays(hw + [None]), _arrays(hg + [hg[0]])     # trailing NULL param is skipped
    sa = (ctypes.c_uint * (len(SIZES) + 1))(*SIZES, SIZES[0])
    eng.lib.SGDBatch(pa, ga, sa, len(SIZES) + 1, 0.05, 1.0)
    for h, w, g in zip(hw, ws, gs):
        assert rel_err(download(eng, h, w.shape), K.sgd(w, g, 0.05, 1.0)) <= 1e-6
    release(eng, *hw, *hg)


@pytest.mark.parametrize("max_norm", [1.0, 1e6])
def test_sgd_batch_clipped(eng, max_norm, policy):
    ws, gs = _param_set(2, SIZES)
    hw, hg = [upload(eng, w) for w in ws], [upload(eng, g) for g in gs]
    sa = (ctypes.c_uint * len(SIZES))(*SIZES)
    norm = eng.lib.SGDBatchClipped(_arrays(hw), _arrays(hg), sa, len(SIZES), 0.1, max_norm)
    n_ref, scale = K.grad_norm_scale(gs, max_norm)
    assert abs(norm - n_ref) <= 1e-5 * n_ref
    for h, w, g in zip(hw, ws, gs):
        assert rel_err(download(eng, h, w.shape), K.sgd_clipped(w, g, 0.1, scale)) <= 1e-6
    release(eng, *hw, *hg)


def test_clip_grad_norm(eng, policy):
    _, gs = _param_set(3, SIZES)
    hg = [upload(eng, g) for g in gs]
    sa = (ctypes.c_uint * len(SIZES))(*SIZES)
    norm = eng.lib.ClipGradNorm(_arrays(hg), sa, len(SIZES), 1.0)
    n_ref, scale = K.grad_norm_scale(gs, 1.0)
    assert abs(norm - n_ref) <= 1e-5 * n_ref
    for h, g in zip(hg, gs):
        assert rel_err(download(eng, h, g.shape), g.astype(np.float64) * scale) <= 1e-6
    release(eng, *hg)


@pytest.mark.parametrize("wd,clip", [(0.01, 1.0), (0.0, 1e30)])
def test_adam_batch_and_shader(eng, wd, clip, policy):
    ws, gs = _param_set(4, SIZES)
    r = rng(5)
    ms = [(0.1 * r.standard_normal(n)).astype(np.float32) for n in SIZES]
    vs = [(0.1 * r.random(n)).astype(np.float32) for n in SIZES]
    lr, b1, b2, eps, t = 1e-3, 0.9, 0.999, 1e-8, 3
    step = K.adam_step_size(lr, b1, b2, t)
    # The kernel receives every hyper-parameter as a float32 (the shader's
    # constant buffer); the oracle is fed the same float32 values, so e.g.
    # 1 - beta2 carries the same rounding as in nn_adam.hlsl.
    f32 = lambda v: float(np.float32(v))
    o_step, o_b1, o_b2, o_eps, o_wd = f32(step), f32(b1), f32(b2), f32(eps), f32(lr * wd)
    hw, hg, hm, hv = ([upload(eng, a) for a in arrs] for arrs in (ws, gs, ms, vs))
    sa = (ctypes.c_uint * len(SIZES))(*SIZES)
    eng.lib.AdamBatch(_arrays(hw), _arrays(hg), _arrays(hm), _arrays(hv), sa, len(SIZES), step, b1, b2,
                      eps, lr * wd, clip)
    for i in range(len(SIZES)):
        w_r, m_r, v_r = K.adam(ws[i], gs[i], ms[i], vs[i], o_step, o_b1, o_b2, o_eps, o_wd, clip)
        assert rel_err(download(eng, hw[i], ws[i].shape), w_r) <= 1e-6
        assert rel_err(download(eng, hm[i], ms[i].shape), m_r) <= 1e-6
        assert rel_err(download(eng, hv[i], vs[i].shape), v_r) <= 1e-6
    # the single-tensor RunShader("adam") path (nn_adam.hlsl CB layout)
    w2, m2, v2 = upload(eng, ws[5]), upload(eng, ms[5]), upload(eng, vs[5])
    run(eng, "adam", [hg[5]], [w2, m2, v2], SIZES[5], fbits(step), fbits(b1), fbits(b2), fbits(eps),
        fbits(lr * wd), fbits(clip), 0)
    w_r, m_r, v_r = K.adam(ws[5], gs[5], ms[5], vs[5], o_step, o_b1, o_b2, o_eps, o_wd, clip)
    assert rel_err(download(eng, w2, ws[5].shape), w_r) <= 1e-6
    release(eng, *hw, *hg, *hm, *hv, w2, m2, v2)


def _ragged_sizes(seed, count):
    """Seeded tensor sizes for the multi-tensor kernels: 1 to 20000
    elements, with exact multiples of the 4096-element chunk mixed in;
    more tensors than one launch table holds (48) when count > 48."""
    r = np.random.default_rng(seed)
    sizes = [int(v) for v in r.integers(1, 20000, count)]
    for i in range(0, count, 7):
        sizes[i] = 4096 * int(r.integers(1, 4))
    return sizes


@pytest.mark.parametrize("seed,count", [(11, 5), (12, 47), (13, 49), (14, 101)])
def test_optimisers_ragged_tensor_lists(eng, seed, count):
    """SGDBatch, AdamBatch and ClipGradNorm over seeded ragged tensor lists,
    across launch-table boundaries, against the float64 oracle."""
    sizes = _ragged_sizes(seed, count)
    sa = (ctypes.c_uint * count)(*sizes)
    ws, gs = _param_set(seed, sizes)
    hw, hg = [upload(eng, w) for w in ws], [upload(eng, g) for g in gs]
    eng.lib.SGDBatch(_arrays(hw), _arrays(hg), sa, count, 0.05, 1.0)
    for h, w, g in zip(hw, ws, gs):
        assert rel_err(download(eng, h, w.shape), K.sgd(w, g, 0.05, 1.0)) <= 1e-6
    release(eng, *hw)
    r = rng(seed + 100)
    ws = [r.standard_normal(n).astype(np.float32) for n in sizes]
    ms = [(0.1 * r.standard_normal(n)).astype(np.float32) for n in sizes]
    vs = [(0.1 * r.random(n)).astype(np.float32) for n in sizes]
    lr, b1, b2, eps, wd, clip, t = 1e-3, 0.9, 0.999, 1e-8, 0.01, 1.0, 2
    step = K.adam_step_size(lr, b1, b2, t)
    f32 = lambda v: float(np.float32(v))
    hw, hm, hv = ([upload(eng, a) for a in arrs] for arrs in (ws, ms, vs))
    eng.lib.AdamBatch(_arrays(hw), _arrays(hg), _arrays(hm), _arrays(hv), sa, count, step, b1, b2,
                      eps, lr * wd, clip)
    for i in range(count):
        w_r, m_r, v_r = K.adam(ws[i], gs[i], ms[i], vs[i], f32(step), f32(b1), f32(b2), f32(eps),
                               f32(lr * wd), clip)
        assert rel_err(download(eng, hw[i], ws[i].shape), w_r) <= 1e-6
        assert rel_err(download(eng, hm[i], ms[i].shape), m_r) <= 1e-6
        assert rel_err(download(eng, hv[i], vs[i].shape), v_r) <= 1e-6
    norm = eng.lib.ClipGradNorm(_arrays(hg), sa, count, 1.0)
    n_ref, scale = K.grad_norm_scale(gs, 1.0)
    assert abs(norm - n_ref) <= 1e-5 * n_ref
    for h, g in zip(hg, gs):
        assert rel_err(download(eng, h, g.shape), g.astype(np.float64) * scale) <= 1e-6
    release(eng, *hw, *hg, *hm, *hv)


def test_adam_batch_counted(eng, policy):
    """AdamBatchCounted keeps t and the step size on the device: t > 0 sets
    the counter and stores the host's step size unchanged (an eager step is
    bit for bit the reference's nn_engine.py:2219-2220 float), t == 0 advances
    the counter and evaluates the step size on the device (within one float
    ulp of the host formula; the stepSize argument is ignored).  The update
    equals AdamBatch with the stored step size, bit for bit."""
    ws, gs = _param_set(6, SIZES)
    r = rng(7)
    ms = [(0.1 * r.standard_normal(n)).astype(np.float32) for n in SIZES]
    vs = [(0.1 * r.random(n)).astype(np.float32) for n in SIZES]
    lr, b1, b2, eps, wd, clip = 1e-3, 0.9, 0.999, 1e-8, 0.01, 1.0
    sa = (ctypes.c_uint * len(SIZES))(*SIZES)
    a = [[upload(eng, x) for x in arrs] for arrs in (ws, gs, ms, vs)]   # counted
    b = [[upload(eng, x) for x in arrs] for arrs in (ws, gs, ms, vs)]   # host step size
    state = upload(eng, np.zeros(2, np.float32))
    for t_arg, t in ((5, 5), (0, 6), (0, 7), (2, 2), (0, 3), (1000, 1000)):
        step = K.adam_step_size(lr, b1, b2, t)
        host = float(np.float32(step)) if t_arg else 123.0      # ignored when t_arg == 0
        eng.lib.AdamBatchCounted(*(_arrays(h) for h in a), sa, len(SIZES), state, t_arg, host, lr,
                                 b1, b2, eps, lr * wd, clip)
        st = download(eng, state, (2,))
        assert int(st[:1].view(np.uint32)[0]) == t
        if t_arg:
            assert st[1] == np.float32(step), (t, st[1], step)
        else:
            assert abs(float(st[1]) - float(np.float32(step))) <= 2.0 ** -23 * step, (t, st[1], step)
        eng.lib.AdamBatch(*(_arrays(h) for h in b), sa, len(SIZES), float(st[1]), b1, b2, eps, lr * wd,
                          clip)
        for i in range(len(SIZES)):
            for j in (0, 2, 3):
                assert np.array_equal(download(eng, a[j][i], (SIZES[i],)),
                                      download(eng, b[j][i], (SIZES[i],))), (t, i, j)
    eng.lib.ClearLastError()
    short = upload(eng, np.zeros(1, np.float32))
    eng.lib.AdamBatchCounted(*(_arrays(h) for h in a), sa, len(SIZES), short, 1, 1e-3, lr, b1, b2, eps,
                             0.0, clip)
    assert "2 floats" in eng.last_error()
    release(eng, *[h for arrs in a + b for h in arrs], state, short)


def test_norm_clip_shaders(eng):
    """grad_sq_reduce per tensor + grad_norm_final + sgd_clipped (the
    dispatches SGDBatchClipped makes in the reference, engine.cpp:514-598)."""
    ws, gs = _param_set(6, [1000, 4097])
    hw, hg = [upload(eng, w) for w in ws], [upload(eng, g) for g in gs]
    parts = (1000 + 255) // 256 + (4097 + 255) // 256
    hp, hns = new(eng, parts), new(eng, 2)
    run(eng, "grad_sq_reduce", [hg[0]], [hp], 1000, 0)
    run(eng, "grad_sq_reduce", [hg[1]], [hp], 4097, (1000 + 255) // 256)
    run(eng, "grad_norm_final", [hp], [hns], parts, fbits(1.0))
    n_ref, scale = K.grad_norm_scale(gs, 1.0)
    ns = download(eng, hns, (2,))
    assert abs(ns[0] - n_ref) <= 1e-5 * n_ref and abs(ns[1] - scale) <= 1e-5 * scale
    for i in range(2):
        run(eng, "sgd_clipped", [hg[i], hns], [hw[i]], ws[i].size, fbits(0.1))
        assert rel_err(download(eng, hw[i], ws[i].shape), K.sgd_clipped(ws[i], gs[i], 0.1, scale)) <= 1e-5
    hs = upload(eng, ws[0])
    run(eng, "sgd", [hg[0]], [hs], 1000, fbits(0.05), fbits(0.5), 0)
    assert rel_err(download(eng, hs, (1000,)), K.sgd(ws[0], gs[0], 0.05, 0.5)) <= 1e-6
    release(eng, *hw, *hg, hp, hns, hs)


# ------------------------------------------------- im2col path (RunShader)
def test_im2col_col2im_reshapes(eng):
    B, C, H, W, k, s, p, OC = 2, 3, 7, 6, 3, 2, 1, 4
    OH, OW = K.conv_out_hw(H, W, k, s, p)
    r = rng(9)
    x = r.standard_normal((B, C, H, W)).astype(np.float32)
    hx, hcol = upload(eng, x), new(eng, C * k * k * B * OH * OW)
    cb = (B, C, H, W, k, s, p, OH, OW)
    run(eng, "im2col", [hx], [hcol], *cb)
    col = download(eng, hcol, (C * k * k, B * OH * OW))
    assert np.array_equal(col, K.im2col(x, k, s, p).astype(np.float32))
    hdx = new(eng, x.size)
    run(eng, "col2im", [hcol], [hdx], *cb)
    assert rel_err(download(eng, hdx, x.shape), K.col2im(col, x.shape, k, s, p)) <= 1e-6
    mm = r.standard_normal((OC, B * OH * OW)).astype(np.float32)
    bias = r.standard_normal(OC).astype(np.float32)
    hmm, hb, hy = upload(eng, mm), upload(eng, bias), new(eng, B * OC * OH * OW)
    for act in (0, 1, 2):
        run(eng, "conv_reshape", [hmm, hb], [hy], B, OC, OH, OW, act)
        z = mm.astype(np.float64) + bias[:, None]
        z = np.maximum(z, 0) if act == 1 else (np.tanh(z) if act == 2 else z)
        assert rel_err(download(eng, hy, (B, OC, OH, OW)), z.reshape(OC, B, OH, OW).transpose(1, 0, 2, 3)) <= 1e-6
    dz = r.standard_normal((B, OC, OH, OW)).astype(np.float32)
    y = r.standard_normal((B, OC, OH, OW)).astype(np.float32)
    hdz, hyy, hG = upload(eng, dz), upload(eng, y), new(eng, dz.size)
    run(eng, "conv_grad_reshape", [hdz], [hG], B, 0, 0, 0, OC, 0, 0, OH, OW)
    assert np.array_equal(download(eng, hG, (OC, B * OH * OW)), K.conv_grad_reshape(dz).astype(np.float32))
    run(eng, "conv_grad_reshape_relu", [hdz, hyy], [hG], B, 0, 0, 0, OC, 0, 0, OH, OW)
    assert np.array_equal(download(eng, hG, (OC, B * OH * OW)), K.conv_grad_reshape(dz, y, 1).astype(np.float32))
    for flags in range(4):
        Mm, Kk, Nn = 5, 9, 7
        a = r.standard_normal(Mm * Kk).astype(np.float32)
        b = r.standard_normal(Kk * Nn).astype(np.float32)
        ha, hb2, hc = upload(eng, a), upload(eng, b), new(eng, Mm * Nn)
        for name in ("matmul_universal", "matmul_heavy", "matmul_reduce"):
            run(eng, name, [ha, hb2], [hc], Mm, Kk, Nn, flags)
            assert rel_err(download(eng, hc, (Mm, Nn)), K.matmul(a, b, Mm, Kk, Nn, flags)) <= 1e-5
        release(eng, ha, hb2, hc)
    release(eng, hx, hcol, hdx, hmm, hb, hy, hdz, hyy, hG)


@pytest.mark.parametrize("M,Kd,N", [(5, 9, 7), (130, 67, 129), (64, 300, 64)])
def test_run_mm(eng, M, Kd, N):
    """nn_engine._run_mm (nn_engine.py:887-893): the flagged GEMM into a
    caller's buffer, through the small- and large-output shader names, for
    every transpose flag, against the float64 oracle."""
    r = rng(M * 7 + Kd)
    a = r.standard_normal(M * Kd).astype(np.float32)
    b = r.standard_normal(Kd * N).astype(np.float32)
    ha, hb, hc = upload(eng, a), upload(eng, b), new(eng, M * N)
    for flags in range(4):
        eng._run_mm(ha, hb, hc, M, Kd, N, flags)
        assert rel_err(download(eng, hc, (M, N)), K.matmul(a, b, M, Kd, N, flags)) <= TOL
    release(eng, ha, hb, hc)


def test_profiler_device_time(eng, capsys):
    """nn_engine.profiler keeps the reference's profiler calls
    (nn_engine.py:183-306: install, enable, report, reset, disable,
    uninstall) and reports each kernel family's launches and GPU time."""
    n = 4096
    r = rng(77)
    hg, hx, ho = upload(eng, r.standard_normal(n).astype(np.float32)), \
        upload(eng, r.standard_normal(n).astype(np.float32)), new(eng, n)
    p = eng.profiler
    p.install()
    p.enable()
    for _ in range(3):
        run(eng, "relu_grad", [hg, hx], [ho], n)
    st = p.stats()
    assert st["relu_grad"][0] == 3 and st["relu_grad"][1] > 0
    p.report("test")
    out = capsys.readouterr().out
    assert "relu_grad" in out and "TOTAL" in out
    p.reset()
    assert "relu_grad" not in p.stats()
    # a whole ConvBackwardFused call is recorded as conv_bwd and its kernels
    # under their own families: the report's percentages still add up to 100
    x = eng.Tensor(r.standard_normal((2, 8, 12, 12)).astype(np.float32), requires_grad=True, track=False)
    w = eng.Tensor((r.standard_normal((16, 8, 3, 3)) * 0.2).astype(np.float32), requires_grad=True,
                   track=False)
    b = eng.Tensor(np.zeros(16, np.float32), requires_grad=True, track=False)
    eng.conv2d(x, w, b, 1, 1, 1).backward()          # seed = ones (nn_engine.py:575-603)
    st = p.stats()
    assert "conv_bwd" in st and "conv_dw" in st
    rows, aggs, (_, total) = p.table(st)
    assert [a[0] for a in aggs] == ["conv_bwd"] and "conv_bwd" not in [q[0] for q in rows]
    assert abs(sum(q[3] for q in rows) - 100.0) < 1e-6
    assert total < sum(ms for _, ms in st.values())
    eng.end_batch()
    p.disable()
    p.uninstall()
    release(eng, hg, hx, ho)


def test_run_sequence(eng):
    """RunSequence replays SeqCmd records (engine.cpp:952-966) built with ResolveShader."""
    from directcompute_torch_amd._lib import SeqCmd
    n = 1000
    g = rng(10).standard_normal(n).astype(np.float32)
    x = rng(11).standard_normal(n).astype(np.float32)
    hg, hx, ho, hw = upload(eng, g), upload(eng, x), new(eng, n), upload(eng, x)
    cmds = (SeqCmd * 2)()
    cmds[0].shader = eng.lib.ResolveShader(b"relu_grad")
    cmds[0].srvs[0], cmds[0].srvs[1], cmds[0].srvCount = hg, hx, 2
    cmds[0].uavs[0], cmds[0].uavCount = ho, 1
    struct.pack_into("I", cmds[0].cbData, 0, n)
    cmds[0].cbSize = 16
    cmds[1].shader = None  # skipped
    eng.lib.RunSequence(ctypes.byref(cmds), 2)
    assert rel_err(download(eng, ho, (n,)), K.relu_grad(g, x)) <= 1e-6
    sa = (ctypes.c_uint * 1)(n)
    eng.lib.RunSequenceWithSGD(ctypes.byref(cmds), 1, _arrays([hw]), _arrays([ho]), sa, 1, 0.1, 1.0)
    assert rel_err(download(eng, hw, (n,)), K.sgd(x, K.relu_grad(g, x), 0.1, 1.0)) <= 1e-6
    # a shader pointer that is not a registry entry is refused before it is
    # read: one inside the table but between entries, and host memory
    before = download(eng, ho, (n,))
    junk = (ctypes.c_char * 64)()
    for bogus in (cmds[0].shader + 1, ctypes.addressof(junk)):
        cmds[0].shader = bogus
        eng.lib.ClearLastError()
        eng.lib.RunSequence(ctypes.byref(cmds), 1)
        assert "unresolved shader pointer" in eng.last_error()
    assert np.array_equal(download(eng, ho, (n,)), before)
    release(eng, hg, hx, ho, hw)
