"""ComputeGraph (nn_engine.py:2505-2771): one training step recorded as a HIP
graph through BeginCapture / EndCapture and replayed with new batches.  Every
replay is compared bit-exactly with the same step run eagerly on a second copy
of the parameters (the step's kernels are deterministic: no atomics), with
SyncGPU and read-backs between the replays, and every replayed step is
checked against the float64 oracle -- softmax-CE with SGD and with AdamW
(whose step count must advance per replay), and Dice with the global norm
clip and Adam."""
import numpy as np
import pytest

from tests import workloads as WL
from tests.helpers import rel_err, rng

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


def _opt(eng, kind, params):
    if kind == "sgd":
        return eng.SGD(params, lr=0.01)
    if kind == "adamw":
        return eng.AdamW(params, lr=1e-3, weight_decay=0.01)
    return eng.Adam(params, lr=1e-3)


def _loss_fn(eng, kind):
    return None if kind == "ce" else eng.dice_loss


def _labels(kind, shape, ncls, seed):
    if kind == "ce":
        return rng(seed).integers(0, ncls, shape[0]).astype(np.float32)
    B, _, H, W = shape
    blobs = (rng(seed).random((B, 1, H // 8, W // 8)) < 0.3).astype(np.float32)
    return np.repeat(np.repeat(blobs, 8, axis=2), 8, axis=3)


def _eager_step(eng, be, net, opt, x, y, clip, loss_kind, max_norm, pins=False):
    """The traced step run eagerly on a second copy of the parameters.
    Returns the loss (mean for a per-sample loss), the network output and,
    with pins=True, what the oracle needs: the device's discrete decisions
    and its gradients before and after the norm clip."""
    opt.zero_grad()
    be.x = eng.Tensor(x, track=True)
    out = _forward(be, net)(be.x)
    fn = _loss_fn(eng, loss_kind) or eng.softmax_ce
    loss = fn(out, eng.Tensor(y, track=True))
    extra = {}
    if pins:
        extra["pins"] = dict(pool_indices=be.pool_indices(), decisions=be.decisions())
    loss.backward()
    if pins:
        extra["grads"] = be.grads()
    if max_norm is not None:
        extra["norm"] = eng.clip_grad_norm(list(be.P.values()), max_norm)
        if pins:
            extra["clipped"] = be.grads()
    opt.step(clip=clip)
    lv = loss.sync()
    res = float(lv[0]) if lv.size == 1 else float(lv.mean()), out.sync().copy(), extra
    eng.end_batch()
    return res


def _check_against_oracle(net, loss_kind, opt_kind, opt, P_before, mv_before, x, y, extra,
                          graph_loss, graph_params, clip, max_norm):
    """One replayed step against the float64 oracle: the loss and gradients
    the oracle computes at the step's starting parameters (taking the device's
    max-pool and ReLU decisions), and the update the optimiser rule gives from
    the device's gradients -- with the step count of this step for Adam."""
    from oracle import kernels as K
    from tests.test_gpu_models import _audit, _compare_grads
    ob = WL.Oracle(P_before, **extra["pins"])
    out = net(ob, x)
    oloss = ob.softmax_ce(out, y) if loss_kind == "ce" else ob.dice(out, y)
    _audit(ob, fwd_tol=1e-5 if loss_kind == "ce" else 4e-5)   # UNet: deep conv + BN chain
    oloss.backward()
    og = ob.grads()
    ref_loss = float(np.mean(oloss.data))
    assert abs(graph_loss - ref_loss) <= 1e-5 * max(1.0, abs(ref_loss))
    _compare_grads(extra["grads"], og)
    g = extra["grads"]
    if max_norm is not None:
        n_ref, _ = K.grad_norm_scale([og[k] for k in sorted(og)], max_norm)
        assert abs(extra["norm"] - n_ref) <= 1e-4 * n_ref
        g = extra["clipped"]
    f32 = lambda v: float(np.float32(v))
    for k in P_before:
        if opt_kind == "sgd":
            w_r = K.sgd(P_before[k], g[k], f32(opt.lr), clip)
        else:
            step = f32(K.adam_step_size(opt.lr, opt.beta1, opt.beta2, opt.t))
            m0, v0 = mv_before[k]
            w_r, _, _ = K.adam(P_before[k], g[k], m0, v0, step, f32(opt.beta1), f32(opt.beta2),
                               f32(opt.eps), f32(opt.lr * opt.weight_decay), clip)
        assert rel_err(graph_params[k], w_r) <= 1e-6, k


def _unet3(be, x):
    return WL.unet(be, x, levels=3)


def _unet3_params(r):
    return WL.unet_params(r, levels=3)


CASES = [
    # name, network, parameters, input shape, classes, loss, optimiser, norm clip
    ("lenet-sgd", WL.lenet, WL.lenet_params, (32, 1, 28, 28), 10, "ce", "sgd", None),
    ("mobilenet-sgd", WL.mobilenet, WL.mobilenet_params, (4, 16, 32, 32), 10, "ce", "sgd", None),
    ("lenet-adamw", WL.lenet, WL.lenet_params, (16, 1, 28, 28), 10, "ce", "adamw", None),
    ("unet-dice-clip-adam", _unet3, _unet3_params, (2, 3, 32, 32), 0, "dice", "adam", 1.0),
]


@pytest.mark.parametrize("name,net,make_params,xshape,ncls,loss_kind,opt_kind,max_norm", CASES,
                         ids=[c[0] for c in CASES])
def test_graph_replay_matches_eager_and_oracle(eng, name, net, make_params, xshape, ncls, loss_kind,
                                               opt_kind, max_norm):
    """Trace one step, replay it on new batches and run the same steps eagerly
    on a second copy of the parameters (with SyncGPU and read-backs between
    them): every replay must equal its eager step bit for bit (loss, output,
    parameters, Adam moments and step count), and every replayed step is
    checked against the float64 oracle."""
    print(f"graph replay case {name} x{xshape}", flush=True)
    P = make_params(rng(5001))
    batches = [(rng(5100 + i).standard_normal(xshape).astype(np.float32)
                if loss_kind == "ce" else rng(5100 + i).random(xshape).astype(np.float32),
                _labels(loss_kind, xshape, ncls, 5200 + i)) for i in range(5)]
    clip = 1.0
    g_be = _Bound(eng, P)
    g_params = list(g_be.P.values())
    g_opt = _opt(eng, opt_kind, g_params)
    e_be = _Bound(eng, P)
    e_opt = _opt(eng, opt_kind, list(e_be.P.values()))
    adam = opt_kind != "sgd"

    def same_state(tag):
        for k in g_be.P:
            assert np.array_equal(g_be.P[k].sync(), e_be.P[k].sync()), f"{tag}: {k}"
        if adam:
            assert g_opt.t == e_opt.t, tag
            for mg, me in zip(g_opt.m + g_opt.v, e_opt.m + e_opt.v):
                assert np.array_equal(mg.sync(), me.sync()), f"{tag}: moments"

    graph = eng.ComputeGraph()
    try:
        graph.trace(_forward(g_be, net), g_opt, batches[0][0], batches[0][1], g_params, clip=clip,
                    loss_fn=_loss_fn(eng, loss_kind), max_norm=max_norm)
        e_loss, e_out, _ = _eager_step(eng, e_be, net, e_opt, *batches[0], clip, loss_kind, max_norm)
        # before any replay the graph's loss / output buffers hold the traced step's values
        assert graph.read_loss() == e_loss
        assert np.array_equal(graph.read_logits(), e_out)
        same_state("trace")
        for i, (x, y) in enumerate(batches[1:4], start=1):
            P_before = e_be.values()
            names = list(e_be.P)
            mv_before = ({k: (e_opt.m[j].sync().copy(), e_opt.v[j].sync().copy())
                          for j, k in enumerate(names)} if adam else None)
            graph.replay(x, y)
            e_loss, e_out, extra = _eager_step(eng, e_be, net, e_opt, x, y, clip, loss_kind,
                                               max_norm, pins=True)
            eng.lib.SyncGPU()
            assert graph.read_loss() == e_loss, f"replay {i}: loss"
            assert np.array_equal(graph.read_logits(), e_out), f"replay {i}: output"
            same_state(f"replay {i}")
            _check_against_oracle(net, loss_kind, opt_kind, e_opt, P_before, mv_before, x, y, extra,
                                  graph.read_loss(), g_be.values(), clip, max_norm)
        # two replays back to back, no host work in between
        for x, y in batches[3:5]:
            graph.replay(x, y)
        for x, y in batches[3:5]:
            _eager_step(eng, e_be, net, e_opt, x, y, clip, loss_kind, max_norm)
        same_state("back-to-back")
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
