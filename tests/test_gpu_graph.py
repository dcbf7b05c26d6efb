"""ComputeGraph (nn_engine.py:2505-2771): one training step recorded as a HIP
graph through BeginCapture / EndCapture and replayed with new batches.  Every
replay is compared bit-exactly with the same step run eagerly on a second copy
of the parameters; the eager steps run between the replays on the same stream,
with SyncGPU and read-backs in between.  The step's kernels are deterministic
(no atomics), so a replay must reproduce the eager bits."""
import numpy as np
import pytest

from tests import workloads as WL
from tests.helpers import rng

pytestmark = pytest.mark.gpu


class _Bound(WL.Device):
    """Device backend whose network input is a given device tensor."""

    def __init__(self, nn, params):
        super().__init__(nn, params)
        self.x = None

    def input(self, a):
        return self.x


def _forward(be, net):
    def fn(xb):
        be.x = xb
        be.mask_nodes.clear()
        be.pool_nodes.clear()
        return net(be, None)
    return fn


def _eager_step(eng, be, net, opt, x, y, clip):
    opt.zero_grad()
    be.x = eng.Tensor(x, track=True)
    logits = _forward(be, net)(be.x)
    loss = eng.softmax_ce(logits, eng.Tensor(y, track=True))
    loss.backward()
    opt.step(clip=clip)
    out = float(loss.sync()[0]), logits.sync().copy()
    eng.end_batch()
    return out


CASES = [
    ("lenet", WL.lenet, WL.lenet_params, (32, 1, 28, 28), 10),
    ("mobilenet", WL.mobilenet, WL.mobilenet_params, (4, 16, 32, 32), 10),
]


@pytest.mark.parametrize("name,net,make_params,xshape,ncls", CASES, ids=[c[0] for c in CASES])
def test_graph_replay_matches_eager(eng, name, net, make_params, xshape, ncls):
    print(f"graph replay case {name} x{xshape}", flush=True)
    P = make_params(rng(5001))
    batches = [(rng(5100 + i).standard_normal(xshape).astype(np.float32),
                rng(5200 + i).integers(0, ncls, xshape[0]).astype(np.float32)) for i in range(5)]
    clip = 1.0
    g_be = _Bound(eng, P)
    g_params = list(g_be.P.values())
    g_opt = eng.SGD(g_params, lr=0.01)
    e_be = _Bound(eng, P)
    e_opt = eng.SGD(list(e_be.P.values()), lr=0.01)

    graph = eng.ComputeGraph()
    try:
        graph.trace(_forward(g_be, net), g_opt, batches[0][0], batches[0][1], g_params, clip=clip)
        e_loss, e_logits = _eager_step(eng, e_be, net, e_opt, batches[0][0], batches[0][1], clip)
        # before any replay the graph's loss/logits buffers hold the traced step's values
        assert graph.read_loss() == e_loss
        assert np.array_equal(graph.read_logits(), e_logits)
        for k in g_be.P:
            assert np.array_equal(g_be.P[k].sync(), e_be.P[k].sync()), k
        for i, (x, y) in enumerate(batches[1:], start=1):
            graph.replay(x, y)
            e_loss, e_logits = _eager_step(eng, e_be, net, e_opt, x, y, clip)
            eng.lib.SyncGPU()
            assert graph.read_loss() == e_loss, f"replay {i}: loss"
            assert np.array_equal(graph.read_logits(), e_logits), f"replay {i}: logits"
            for k in g_be.P:
                assert np.array_equal(g_be.P[k].sync(), e_be.P[k].sync()), f"replay {i}: {k}"
        # two replays back to back, no host work in between
        for x, y in batches[1:3]:
            graph.replay(x, y)
            _eager_step(eng, e_be, net, e_opt, x, y, clip)
        for k in g_be.P:
            assert np.array_equal(g_be.P[k].sync(), e_be.P[k].sync()), f"back-to-back: {k}"
    finally:
        graph.release()
        eng.end_batch()


def test_capture_refuses_readback(eng):
    """A read-back inside the recorded step makes EndCapture fail with the
    reason; the engine is usable afterwards and the held buffers are returned."""
    lib = eng.lib
    assert lib.BeginCapture()
    assert not lib.BeginCapture()  # one capture at a time
    t = eng.Tensor(np.arange(16, dtype=np.float32), track=False)  # small upload: recorded
    u = eng.relu(t)
    out = np.empty(16, np.float32)
    import ctypes
    lib.ReadBuffer(u.gpu_buf, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    assert not lib.EndCapture()
    assert "ReadBuffer" in eng.last_error()
    eng.end_batch()
    del u, t
    v = eng.relu(eng.Tensor(np.linspace(-1, 1, 1000, dtype=np.float32)))
    assert np.array_equal(v.sync(), np.maximum(np.linspace(-1, 1, 1000, dtype=np.float32), 0))
    eng.end_batch()
    assert not lib.EndCapture()  # nothing open
