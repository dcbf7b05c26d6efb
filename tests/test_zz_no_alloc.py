"""ClipGradNormNoAlloc: the norm clip that allocates nothing, against
ClipGradNorm (the entry point whose kernels it shares, nn_engine.py:1335-1355
for the reference's clip_grad_norm).

Both run the same kernels in the same order, so the norm and every clipped
gradient must agree bit for bit.  Two calls in a row, the second over fewer
and smaller tensors, show that nothing left in the shared static scratch
leaks into the next call.  The refusal of a request beyond the scratch's
65536 partial sums is checked with one small handle repeated so often that
its chunks exceed that count (the host refuses it before any launch)."""
import ctypes

import numpy as np
import pytest

from tests.helpers import download, release, rng, upload

pytestmark = pytest.mark.gpu

MAX_PARTS = 65536
CHUNK = 4096


def _arrays(handles, sizes):
    n = len(handles)
    return (ctypes.c_void_p * n)(*handles), (ctypes.c_uint * n)(*sizes)


def _clip(eng, fn, grads, max_norm):
    """Upload `grads`, clip them with `fn`, return (norm, clipped arrays)."""
    hs = [upload(eng, g) for g in grads]
    try:
        ga, sa = _arrays(hs, [g.size for g in grads])
        norm = fn(ga, sa, len(hs), max_norm)
        assert eng.last_error() == "", eng.last_error()
        return norm, [download(eng, h, g.shape) for h, g in zip(hs, grads)]
    finally:
        release(eng, *hs)


@pytest.mark.parametrize("max_norm", [0.5, 1e6], ids=["clipped", "unclipped"])
def test_noalloc_clip_matches_clip_grad_norm(eng, max_norm):
    print(f"no-alloc clip, max_norm={max_norm}", flush=True)
    r = rng(7100)
    # first call: ragged tensors, one larger than a chunk table's worth
    first = [r.standard_normal(n).astype(np.float32) for n in (1, 4095, 4097, 300_001, 61, 2_000_000)]
    # second call: fewer, smaller tensors
    second = [r.standard_normal(n).astype(np.float32) for n in (5, 1000, 8193)]
    for grads in (first, second):
        eng.lib.ClearLastError()
        n_ref, g_ref = _clip(eng, eng.lib.ClipGradNorm, grads, max_norm)
        n_new, g_new = _clip(eng, eng.lib.ClipGradNormNoAlloc, grads, max_norm)
        exact = np.sqrt(sum(float(np.sum(g.astype(np.float64) ** 2)) for g in grads))
        assert abs(n_ref - exact) <= 1e-6 * exact
        assert n_new == n_ref
        for a, b in zip(g_new, g_ref):
            assert np.array_equal(a, b)
        if max_norm < exact:
            scale = np.float32(max_norm) / np.float32(n_ref + np.float32(1e-6))
            assert np.allclose(g_new[0], grads[0] * scale, rtol=1e-6, atol=0)
        else:
            for a, g in zip(g_new, grads):
                assert np.array_equal(a, g)


def test_noalloc_clip_many_tensors_and_nulls(eng):
    """More tensors than one launch table holds (48), with NULL entries."""
    print("no-alloc clip, 130 tensors with NULLs", flush=True)
    r = rng(7101)
    grads = [r.standard_normal(int(n)).astype(np.float32) for n in r.integers(1, 9000, 130)]
    hs = [upload(eng, g) for g in grads]
    try:
        live = [h if i % 7 else None for i, h in enumerate(hs)]
        sizes = [g.size for g in grads]
        ga, sa = _arrays(live, sizes)
        ref_hs = [upload(eng, g) for g in grads]
        rga, _ = _arrays([h if i % 7 else None for i, h in enumerate(ref_hs)], sizes)
        n_ref = eng.lib.ClipGradNorm(rga, sa, len(hs), 1.0)
        n_new = eng.lib.ClipGradNormNoAlloc(ga, sa, len(hs), 1.0)
        assert n_new == n_ref
        for i, (h, rh, g) in enumerate(zip(hs, ref_hs, grads)):
            a, b = download(eng, h, g.shape), download(eng, rh, g.shape)
            assert np.array_equal(a, b), i
            if i % 7 == 0:
                assert np.array_equal(a, g), i   # NULL entries are untouched
        release(eng, *ref_hs)
    finally:
        release(eng, *hs)


def test_noalloc_clip_refuses_beyond_scratch(eng):
    print("no-alloc clip, request beyond the static scratch", flush=True)
    g = np.ones(CHUNK, np.float32)
    h = upload(eng, g)
    try:
        n = MAX_PARTS + 1      # one chunk each: one partial too many
        ga, sa = _arrays([h] * n, [CHUNK] * n)
        eng.lib.ClearLastError()
        assert eng.lib.ClipGradNormNoAlloc(ga, sa, n, 1.0) == -1.0
        assert "static scratch" in eng.last_error()
        assert np.array_equal(download(eng, h, g.shape), g)   # nothing ran
        # exactly at the limit it runs (the same handle, summed MAX_PARTS times)
        eng.lib.ClearLastError()
        norm = eng.lib.ClipGradNormNoAlloc(ga, sa, MAX_PARTS, 1e9)
        assert eng.last_error() == ""
        assert norm == pytest.approx(np.sqrt(float(MAX_PARTS * CHUNK)), rel=1e-6)
    finally:
        release(eng, h)


def test_noalloc_clip_under_capture_and_no_pool_use(eng):
    """The property the entry point exists for: it allocates nothing.  An
    eager call leaves the buffer pool's counters and held bytes unchanged,
    and a call recorded between BeginCapture and EndCapture (where the engine
    refuses allocations and read-backs, so an allocating call would fail the
    capture) returns NaN, records a graph, and every replay of that graph
    clips like an eager ClipGradNorm on the same gradients, bit for bit."""
    print("no-alloc clip, pool counters and graph capture", flush=True)
    lib = eng.lib
    r = rng(7102)
    grads = [(3 * r.standard_normal(n)).astype(np.float32) for n in (4097, 300, 70_001)]
    sizes = [g.size for g in grads]
    hs = [upload(eng, g) for g in grads]
    ref = [upload(eng, g) for g in grads]
    try:
        ga, sa = _arrays(hs, sizes)
        rga, _ = _arrays(ref, sizes)
        # eager: no pool request, nothing newly held
        lib.SyncGPU()
        lib.ResetPoolStats()
        held = lib.GetPoolMemory()
        eng.lib.ClearLastError()
        n_eager = lib.ClipGradNormNoAlloc(ga, sa, len(hs), 1.0)
        assert eng.last_error() == "" and n_eager > 1.0
        assert eng.get_pool_stats() == (0, 0) and lib.GetPoolMemory() == held
        # recorded
        for h, g in zip(hs, grads):
            lib.UpdateBuffer(h, g.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        assert lib.BeginCapture()
        assert np.isnan(lib.ClipGradNormNoAlloc(ga, sa, len(hs), 1.0))
        graph = lib.EndCapture()
        assert graph, eng.last_error()
        try:
            for rep in range(3):
                # eager work between replays: restore the inputs, clip the
                # reference copies with the allocating entry point
                for h, rh, g in zip(hs, ref, grads):
                    lib.UpdateBuffer(h, g.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
                    lib.UpdateBuffer(rh, g.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
                n_ref = lib.ClipGradNorm(rga, sa, len(ref), 1.0)
                assert n_ref == n_eager
                assert lib.ReplayGraph(graph), eng.last_error()
                lib.SyncGPU()
                for h, rh, g in zip(hs, ref, grads):
                    a, b = download(eng, h, g.shape), download(eng, rh, g.shape)
                    assert np.array_equal(a, b), rep
                    assert not np.array_equal(a, g)            # the replay clipped
        finally:
            lib.ReleaseGraph(graph)
    finally:
        release(eng, *hs, *ref)
