"""Whole training steps of the benchmark networks through the drop-in
nn_engine API on the GPU, compared with the float64 oracle: loss, every
parameter gradient (max|g - g_ref| / max|g_ref| <= 1e-4) and the optimiser
update.  The oracle takes every discrete decision from the device run: the
max-pool argmax indices (compared bit-exactly against the oracle's own scan in
test_gpu_kernels.py) and the ReLU / ReLU6 masks.  A float32 activation within
round-off of a tie or of 0 could otherwise send a gradient down a different
path than the float64 forward chooses.  Every adopted decision is audited
against the oracle's own (tests/workloads.py DecisionAudit): a disagreement
must be a near-tie (|z| <= 1e-5 max|z|, or pooled values equal to that
bound), and the device's forward values at the decision sites must match the
oracle's to the same bound."""
import numpy as np
import pytest

from oracle import kernels as K
from tests import workloads as WL
from tests.helpers import TOL, rel_err, rng

pytestmark = pytest.mark.gpu

f32 = lambda v: float(np.float32(v))


def _compare_grads(dev_g, ref_g, tol=TOL):
    """Per-tensor max|g - g_ref| / max|g_ref| <= tol.  A reference that is zero
    up to float64 round-off (< 1e-9 of the largest gradient of the step) is
    analytically zero -- e.g. the bias of a conv feeding a training-mode
    BatchNorm, whose mean subtraction cancels it -- and the device value must
    then be zero up to float32 round-off (<= 1e-5 of the largest gradient)."""
    assert set(dev_g) == set(ref_g), (sorted(dev_g), sorted(ref_g))
    G = max(float(np.max(np.abs(v))) for v in ref_g.values())
    worst = (0.0, None)
    for k in ref_g:
        if float(np.max(np.abs(ref_g[k]))) < 1e-9 * G:
            assert float(np.max(np.abs(dev_g[k]))) <= 1e-5 * G, f"{k}: expected ~0"
            continue
        worst = max(worst, (rel_err(dev_g[k], ref_g[k]), k))
    assert worst[0] <= tol, f"worst gradient {worst[1]}: {worst[0]:.3e}"
    return worst


def _audit(ob, tie_tol=1e-5, fwd_tol=1e-5):
    """Check the oracle's record of the adopted decisions; print the counts."""
    print("  decisions: " + ob.audit.check(tie_tol, fwd_tol), flush=True)


def _run_device(eng, net, params, x, loss_fn):
    be = WL.Device(eng, params)
    out = net(be, x)
    loss = loss_fn(be, out)
    pins = dict(pool_indices=be.pool_indices(), decisions=be.decisions())
    loss.backward()
    return be, loss, pins


def test_lenet_step_sgd(eng):
    """LeNet-5 b64 full step: forward, softmax-CE, backward, SGD lr 0.01 (element clip 1.0)."""
    r = rng(1000)
    x = r.standard_normal((64, 1, 28, 28)).astype(np.float32)
    y = rng(1002).integers(0, 10, 64).astype(np.float32)
    P = WL.lenet_params(rng(1001))
    be, loss, pins = _run_device(eng, WL.lenet, P, x, lambda b, z: b.softmax_ce(z, y))
    lv = float(loss.sync()[0])
    g = be.grads()
    eng.SGD(list(be.P.values()), lr=0.01).step(clip=1.0)
    new = be.values()
    eng.end_batch()

    ob = WL.Oracle(P, **pins)
    oloss = ob.softmax_ce(WL.lenet(ob, x), y)
    _audit(ob)
    oloss.backward()
    og = ob.grads()
    assert abs(lv - float(oloss.data[0])) <= 1e-5 * abs(float(oloss.data[0]))
    _compare_grads(g, og)
    for k in P:  # the update applied to the device's own gradients
        assert rel_err(new[k], K.sgd(P[k], g[k], f32(0.01), 1.0)) <= 1e-6, k


def test_lenet_gradient_accumulation(eng):
    """Two backward passes without zero_grad accumulate (grad_accum on the
    aliased first gradient, nn_engine.py:605-610; train_alexnet.py accum_steps)."""
    P = WL.lenet_params(rng(7))
    xs = [rng(8 + i).standard_normal((16, 1, 28, 28)).astype(np.float32) for i in range(2)]
    ys = [rng(20 + i).integers(0, 10, 16).astype(np.float32) for i in range(2)]
    be = WL.Device(eng, P)
    pins = []
    for x, y in zip(xs, ys):
        be.pool_nodes, be.mask_nodes = [], []
        loss = be.softmax_ce(WL.lenet(be, x), y)
        pins.append(dict(pool_indices=be.pool_indices(), decisions=be.decisions()))
        loss.backward()
    g = be.grads()
    eng.end_batch()
    total = None
    for x, y, pin in zip(xs, ys, pins):
        ob = WL.Oracle(P, **pin)
        ol = ob.softmax_ce(WL.lenet(ob, x), y)
        _audit(ob)
        ol.backward()
        og = ob.grads()
        total = og if total is None else {k: total[k] + og[k] for k in og}
    _compare_grads(g, total)


@pytest.mark.parametrize("B", [2, 128], ids=["b2", "b128"])
def test_alexnet_step_adamw(eng, B):
    """AlexNet-224 (Linear 9216-4096-4096-1000) full step with AdamW lr 1e-4,
    wd 0.01, element clip 1.0: at batch 2, and at batch 128 -- the timed
    training step itself, with its split-K choices, stride-phase c1 copy and
    tile plans."""
    x = rng(5000).standard_normal((B, 3, 224, 224)).astype(np.float32)
    y = rng(5002).integers(0, 1000, B).astype(np.float32)
    P = WL.alexnet_params(rng(5001))
    be, loss, pins = _run_device(eng, WL.alexnet, P, x, lambda b, z: b.softmax_ce(z, y))
    lv = float(loss.sync()[0])
    g = be.grads()
    params = list(be.P.values())
    opt = eng.AdamW(params, lr=1e-4, weight_decay=0.01)
    opt.step(clip=1.0)
    new = be.values()
    eng.end_batch()

    ob = WL.Oracle(P, **pins)
    oloss = ob.softmax_ce(WL.alexnet(ob, x), y)
    _audit(ob)
    oloss.backward()
    og = ob.grads()
    assert abs(lv - float(oloss.data[0])) <= 1e-5 * abs(float(oloss.data[0]))
    _compare_grads(g, og)
    # The first Adam step is ~lr*sign(g), ill-conditioned where g ~ 0, so the
    # update is checked on the device's own gradients (plumbing: step size,
    # decay, clip, moment buffers).
    step = f32(K.adam_step_size(1e-4, 0.9, 0.999, 1))
    for k in P:
        w_r, _, _ = K.adam(P[k], g[k], np.zeros(P[k].shape), np.zeros(P[k].shape), step, f32(0.9),
                           f32(0.999), f32(1e-8), f32(1e-4 * 0.01), 1.0)
        assert rel_err(new[k], w_r) <= 1e-6, k


@pytest.mark.parametrize("B,S", [(2, 64), (8, 256)], ids=["b2_64", "b8_256"])
def test_unet_step_clip_adam(eng, B, S):
    """UNet-base16 (4 levels, conv3x3-BN-ReLU x2, maxpool, upsample, concat,
    1x1 head, sigmoid, Dice); global-norm clip 1.0 then Adam lr 1e-3.  At
    batch 2 64x64, and at the timed size, batch 8 256x256."""
    x = rng(4000).random((B, 3, S, S)).astype(np.float32)
    blobs = (rng(4002).random((B, 1, S // 8, S // 8)) < 0.3).astype(np.float32)
    t = np.repeat(np.repeat(blobs, 8, axis=2), 8, axis=3)
    P = WL.unet_params(rng(4001))
    be, loss, pins = _run_device(eng, WL.unet, P, x, lambda b, p: b.dice(p, t))
    lv = loss.sync().copy()
    params = list(be.P.values())
    norm = eng.clip_grad_norm(params, 1.0)
    g = be.grads()
    opt = eng.Adam(params, lr=1e-3)
    opt.step(clip=1.0)
    new = be.values()
    eng.end_batch()

    ob = WL.Oracle(P, **pins)
    oloss = ob.dice(WL.unet(ob, x), t)
    # 22 ReLU sites deep through conv + training-mode BN: the float32
    # forward drifts up to about 1e-5 of max|z| by the last decoder layers
    # (measured 1.01e-5 at b8 256^2, 9.2e-6 at b2 64^2)
    _audit(ob, fwd_tol=4e-5)
    oloss.backward()
    og = ob.grads()
    assert rel_err(lv, oloss.data) <= 1e-5
    n_ref, scale = K.grad_norm_scale([og[k] for k in sorted(og)], 1.0)
    assert abs(norm - n_ref) <= 1e-4 * n_ref
    _compare_grads(g, {k: v * scale for k, v in og.items()})
    step = f32(K.adam_step_size(1e-3, 0.9, 0.999, 1))
    for k in P:
        w_r, _, _ = K.adam(P[k], g[k], np.zeros(P[k].shape), np.zeros(P[k].shape), step,
                           f32(0.9), f32(0.999), f32(1e-8), 0.0, 1.0)
        assert rel_err(new[k], w_r) <= 1e-6, k


@pytest.mark.parametrize("B,S", [(2, 32), (64, 112)], ids=["b2_32", "b64_112"])
def test_mobilenet_ir_stack_step(eng, B, S):
    """MobileNetV2 inverted-residual stack (16->24 s2, 24->24, 24->32 s2,
    32->32 x2; BN train mode, ReLU6, depthwise 3x3, residual adds), then GAP +
    Linear + softmax-CE, SGD.  At batch 2 32x32, and at the timed size, batch
    64 112x112 (the float64 oracle needs about 13 GB of host memory)."""
    x = rng(3000).standard_normal((B, 16, S, S)).astype(np.float32)
    y = rng(3002).integers(0, 10, B).astype(np.float32)
    P = WL.mobilenet_params(rng(3001))
    be, loss, pins = _run_device(eng, WL.mobilenet, P, x, lambda b, z: b.softmax_ce(z, y))
    lv = float(loss.sync()[0])
    g = be.grads()
    eng.SGD(list(be.P.values()), lr=0.01).step(clip=1e30)
    new = be.values()
    eng.end_batch()
    ob = WL.Oracle(P, **pins)
    oloss = ob.softmax_ce(WL.mobilenet(ob, x), y)
    _audit(ob)
    oloss.backward()
    og = ob.grads()
    assert abs(lv - float(oloss.data[0])) <= 1e-5 * abs(float(oloss.data[0]))
    _compare_grads(g, og)
    for k in P:
        assert rel_err(new[k], K.sgd(P[k], g[k], f32(0.01), 1e30)) <= 1e-6, k


def test_metrics_epoch(eng):
    """Metrics (nn_engine.py:2336-2385): loss and accuracy accumulated on the
    GPU over several batches of a LeNet forward, read back once by collect().
    The correct count is bit-exact (first-max-wins argmax, ties included);
    the average loss matches the oracle's per-batch CE within float32."""
    P = WL.lenet_params(rng(6001))
    be = WL.Device(eng, P)
    m = eng.Metrics()
    losses, correct, n = [], 0, 0
    for i in range(4):
        B = 16 + 8 * i
        x = rng(6100 + i).standard_normal((B, 1, 28, 28)).astype(np.float32)
        y = rng(6200 + i).integers(0, 10, B).astype(np.float32)
        z = WL.lenet(be, x)
        if i == 2:  # a tied row: the first maximum wins
            zz = z.sync().copy()
            zz[0, :] = 0.0
            z.upload(zz)
        loss = eng.softmax_ce(z, eng.Tensor(y, track=True))
        m.update(loss, z, eng.Tensor(y, track=True))
        zv = z.sync().copy()
        losses.append(K.ce_loss(zv, y))
        correct += K.argmax_correct(zv, y)
        n += B
        eng.end_batch()
    avg, acc = m.collect(n)
    assert acc == correct / n
    assert abs(avg - np.mean(losses)) <= 1e-5 * abs(np.mean(losses))
    m.reset()
    assert m.collect(n) == (0.0, 0.0)
