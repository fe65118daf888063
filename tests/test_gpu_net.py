"""Traced graphs on the GPU through the generic builder (oxh_net_*): the JIT's eager path, the
reference's autograd test on BatchNorm -> reshape -> cross entropy, a general graph with every
op kind, and MobileNetV4-Conv-S assembled from the generic modules against the native trainer.
Every launch of every program is recomputed by the oracle from the device tensors it read."""

import numpy as np
import pytest
import torch

import jit
import nn
import oracle
import oxide_hip as ox
import tensor as tn
import training as T
from helpers import assert_bitexact, assert_close, host
from oracle_checker import OracleChecker

pytestmark = pytest.mark.gpu


def _run_checked(program):
    checker = OracleChecker()
    for op in program.ops:
        checker.before(op)
        op.launch()
        checker.after(op)
    program.check()
    return checker.counts


def test_traced_batch_norm_recomputes_batch_statistics_each_run():
    """jit.rs:763-782 through trace: BatchNorm2d is no plan operation, so the traced graph runs
    eagerly (CompiledPlan::Eager); each run normalizes with its own batch statistics (about
    [-1, 1] for both [1, 3] and [10, 20]) and updates the running statistics as the oracle's
    two training forwards do."""
    layer = nn.BatchNorm2d(1)
    example = np.array([1.0, 3.0], np.float32).reshape(1, 1, 1, 2)
    module = jit.trace([example], lambda i: layer(i[0]))
    first = module.run([example])
    second = module.run([np.array([10.0, 20.0], np.float32).reshape(1, 1, 1, 2)])
    for out in (first, second):
        assert out.shape == (1, 1, 1, 2)
        assert abs(out.ravel()[0] + 1) < 1e-4 and abs(out.ravel()[1] - 1) < 1e-4
    assert module.cached_specializations() == 1
    assert isinstance(module.plan_for(((1, 1, 1, 2),)), jit.EagerPlan)
    rm, rv = np.zeros(1, np.float32), np.ones(1, np.float32)
    one, zero = np.ones(1, np.float32), np.zeros(1, np.float32)
    for x in (example, np.array([10.0, 20.0], np.float32).reshape(1, 1, 1, 2)):
        y, _, _, rm, rv = oracle.bn_forward(x, one, zero, rm, rv)
    assert_close(second.ravel(), y.ravel(), what="second run")
    assert_close(host(layer.state.running_mean), rm, what="running mean")
    assert_close(host(layer.state.running_variance), rv, what="running variance")


def _bn_reshape_ce():
    x = tn.input((3, 2, 1, 1), requires_grad=True)
    w, b = nn.Parameter([1.2, 0.7]), nn.Parameter([0.1, -0.2])
    t = tn.input((3,))
    loss = (x.batch_norm2d(w.tensor(), b.tensor(), tn.BatchNormState(2), True, 0.1, 1e-5)
            .reshape((3, 2)).cross_entropy(t))
    return x, w, b, t, loss


def test_batch_norm_reshape_cross_entropy_gradient_matches_finite_difference():
    """tensor/mod.rs:627-686 through the generic builder: BN (train) -> reshape [3, 2] -> cross
    entropy on data [1, 4, 2, 0, -1, 3], targets [0, 1, 0].  Every launch against the oracle;
    the input gradient equals the oracle's chain (autograd.rs:315-383, 529-554) and the
    central finite difference of device forward runs (step 1e-3, tolerance 2e-3); the weight
    and bias gradients exist."""
    data = np.array([1.0, 4.0, 2.0, 0.0, -1.0, 3.0], np.float32).reshape(3, 2, 1, 1)
    targets = np.array([0.0, 1.0, 0.0], np.float32)
    x, w, b, t, loss = _bn_reshape_ce()
    prog = tn.training_program(loss)
    prog.feed(x, data)
    prog.feed(t, targets)
    counts = _run_checked(prog)
    assert counts == {"batch_norm2d_forward": 1, "cross_entropy": 1,
                      "batch_norm2d_backward": 1}
    analytic = prog.gradient(x).host()
    assert prog.gradient(w.tensor()) is not None and prog.gradient(b.tensor()) is not None
    # the oracle's whole chain on the same inputs
    gamma, beta = np.float32([1.2, 0.7]), np.float32([0.1, -0.2])
    y, mean, inv, _, _ = oracle.bn_forward(data, gamma, beta, np.zeros(2, np.float32),
                                           np.ones(2, np.float32))
    dl = oracle.ce_backward(y.reshape(3, 2), targets, 1.0)
    dx, dw, db = oracle.bn_backward(dl.reshape(3, 2, 1, 1), data, gamma, mean, inv)
    assert_close(analytic, dx, rtol=1e-5, atol=1e-6, what="input gradient")
    assert_close(prog.gradient(w.tensor()).host(), dw, rtol=1e-5, atol=1e-6, what="dweight")
    assert_close(prog.gradient(b.tensor()).host(), db, rtol=1e-5, atol=1e-6, what="dbias")
    # finite differences of device forward runs (fresh running statistics each build)
    fx, _, _, ft, floss = _bn_reshape_ce()
    fwd = tn.forward_program(floss, [fx, ft])
    fwd.feed(ft, targets)

    def device_loss(values):
        fwd.feed(fx, values)
        fwd.run()
        fwd.check()
        return float(fwd.value(floss).host()[0])

    step = 1e-3
    for i in range(data.size):
        pos, neg = data.copy().ravel(), data.copy().ravel()
        pos[i] += step
        neg[i] -= step
        numerical = (device_loss(pos.reshape(data.shape)) -
                     device_loss(neg.reshape(data.shape))) / (2 * step)
        assert abs(analytic.ravel()[i] - numerical) < 2e-3, (i, analytic.ravel()[i], numerical)


def test_general_graph_every_op_matches_oracle():
    """A graph with every op kind the builder takes, some constants and an input requiring a
    gradient: conv (parameter weight, constant bias), eval-mode BatchNorm, ReLU, mul by a
    constant mask, a second consumer of a value (accumulated gradient), average pool, a
    reshape whose input has two consumers (copied gradient), a cross entropy that is not the
    root, the root scaled by a constant.  Every launch against the oracle, the input and
    parameter gradients against torch float64 autograd of the same graph."""
    r = np.random.default_rng(31)
    n, c, h, w = 4, 3, 6, 6
    xv = r.standard_normal((n, c, h, w)).astype(np.float32)
    wv = (r.standard_normal((5, c, 3, 3)) * 0.3).astype(np.float32)
    bv = r.standard_normal(5).astype(np.float32)
    gam, bet = r.uniform(0.5, 1.5, 5).astype(np.float32), r.uniform(-0.2, 0.2, 5).astype(np.float32)
    rm, rv = r.uniform(-0.3, 0.3, 5).astype(np.float32), r.uniform(0.5, 2.0, 5).astype(np.float32)
    mask = (r.uniform(0, 1, (n, 5, h, w)) > 0.3).astype(np.float32) * 1.5
    targets = r.integers(0, 45, n).astype(np.float32)

    x = tn.input((n, c, h, w), requires_grad=True)
    weight = nn.Parameter(wv)
    gamma, beta = nn.Parameter(gam), nn.Parameter(bet)
    state = tn.BatchNormState(5, torch.from_numpy(rm).cuda(), torch.from_numpy(rv).cuda())
    conv = x.conv2d(weight.tensor(), tn.constant(bv), 1, 1, 1)
    a = conv.batch_norm2d(gamma.tensor(), beta.tensor(), state, False, 0.1, 1e-5).relu()
    m = a.mul(tn.constant(mask)).add(a)          # a has two consumers
    pooled = m.avg_pool2d((2, 2), (2, 2))        # [4, 5, 3, 3]
    flat = pooled.reshape((n, 45))
    # 1 x 1 windows keep every value: views of their inputs (no launch); the first one's input
    # has other consumers (its gradient is copied), the second one's only it (the gradient
    # buffer is shared).  other = pooled * pooled
    other = pooled.avg_pool2d((1, 1), (1, 1)).mul(pooled).avg_pool2d((1, 1), (1, 1))
    t = tn.input((n,))
    ce = flat.cross_entropy(t)
    side = other.reshape((n * 45,)).reshape((n, 45)).cross_entropy(t)
    loss = ce.add(side).mul(tn.constant([0.5]))
    prog = tn.training_program(loss)
    prog.feed(x, xv)
    prog.feed(t, targets)
    counts = _run_checked(prog)
    assert counts["avg_pool2d_forward"] == 1, dict(counts)  # the 1 x 1 windows launch nothing
    for kind in ("conv2d_forward", "batch_norm2d_eval_forward", "relu_forward", "mul_forward",
                 "add_forward", "avg_pool2d_forward", "cross_entropy_forward", "seed",
                 "mul_backward", "add_backward", "reshape_backward", "cross_entropy_backward",
                 "avg_pool2d_backward", "relu_backward", "batch_norm2d_eval_backward",
                 "conv2d_backward", "avg_pool2d_view_backward"):
        assert counts[kind] >= 1, (kind, dict(counts))
    # torch float64 autograd of the same graph
    d = lambda v: torch.tensor(v, dtype=torch.float64, requires_grad=True)  # noqa: E731
    tx, tw, tg, tb = d(xv), d(wv), d(gam), d(bet)
    tconv = torch.nn.functional.conv2d(tx, tw, torch.tensor(bv, dtype=torch.float64), 1, 1)
    ta = torch.nn.functional.batch_norm(tconv, torch.tensor(rm, dtype=torch.float64),
                                        torch.tensor(rv, dtype=torch.float64), tg, tb, False,
                                        0.1, 1e-5).relu()
    tm = ta * torch.tensor(mask, dtype=torch.float64) + ta
    tp = torch.nn.functional.avg_pool2d(tm, 2, 2)
    tt = torch.tensor(targets, dtype=torch.long)
    tl = 0.5 * (torch.nn.functional.cross_entropy(tp.reshape(n, 45), tt) +
                torch.nn.functional.cross_entropy((tp * tp).reshape(n, 45), tt))
    tl.backward()
    assert abs(float(prog.value(loss).host()[0]) - tl.item()) <= 1e-5 * abs(tl.item())
    for got, ref, what in ((prog.gradient(x), tx.grad, "dx"), (prog.gradient(weight.tensor()),
                           tw.grad, "dweight"), (prog.gradient(gamma.tensor()), tg.grad, "dgamma"),
                           (prog.gradient(beta.tensor()), tb.grad, "dbeta")):
        ref = ref.numpy()
        np.testing.assert_allclose(got.host(), ref, rtol=1e-4, atol=1e-6 * np.abs(ref).max(),
                                   err_msg=what)
    # running statistics untouched in eval mode; constants get no gradient buffer
    np.testing.assert_array_equal(host(state.running_mean), rm)
    assert prog.gradient(t) is None


def test_shared_parameters_accumulate_every_use():
    """One 1x1 convolution's weight and bias used by two layers, one BatchNorm's gamma and beta
    by three (two after those convolutions, one fused with a depthwise convolution), a
    residual add: every use after a parameter's first adds its gradient into the parameter's
    (the later ones are formed beside the launch's main output and accumulated after it).
    Every launch against the oracle, the gradients against torch float64 autograd."""
    r = np.random.default_rng(47)
    n, c, h, w = 4, 4, 6, 6
    xv = r.standard_normal((n, c, h, w)).astype(np.float32)
    wv = (r.standard_normal((c, c, 1, 1)) * 0.5).astype(np.float32)
    bv = r.standard_normal(c).astype(np.float32)
    dwv = (r.standard_normal((c, 1, 3, 3)) * 0.5).astype(np.float32)
    dbv = r.standard_normal(c).astype(np.float32)
    gam, bet = r.uniform(0.5, 1.5, c).astype(np.float32), r.uniform(-0.2, 0.2, c).astype(np.float32)
    targets = r.integers(0, c * 9, n).astype(np.float32)

    x = tn.input((n, c, h, w), requires_grad=True)
    weight, bias = nn.Parameter(wv), nn.Parameter(bv)
    dweight, dbias = nn.Parameter(dwv), nn.Parameter(dbv)
    gamma, beta = nn.Parameter(gam), nn.Parameter(bet)

    def block(v, wt, b, stride, pad, groups):
        conv = v.conv2d(wt.tensor(), b.tensor(), stride, pad, groups)
        return conv.batch_norm2d(gamma.tensor(), beta.tensor(), tn.BatchNormState(c), True,
                                 0.1, 1e-5)

    a = block(x, weight, bias, 1, 0, 1).relu()
    b2 = block(a, weight, bias, 1, 0, 1).relu()
    s = block(b2, dweight, dbias, 1, 1, c).add(b2)
    t = tn.input((n,))
    loss = s.avg_pool2d((2, 2), (2, 2)).reshape((n, c * 9)).cross_entropy(t)
    prog = tn.training_program(loss)
    prog.feed(x, xv)
    prog.feed(t, targets)
    counts = _run_checked(prog)
    assert counts["side accumulate"] >= 4, dict(counts)
    assert counts["conv2d_backward"] >= 2, dict(counts)

    d = lambda v: torch.tensor(v, dtype=torch.float64, requires_grad=True)  # noqa: E731
    tx, tw, tb, tdw, tdb, tg, tbe = d(xv), d(wv), d(bv), d(dwv), d(dbv), d(gam), d(bet)
    F = torch.nn.functional

    conv_out = []

    def tblock(v, wt, b, pad, groups):
        y = F.conv2d(v, wt, b, 1, pad, 1, groups)
        y.retain_grad()
        conv_out.append(y)
        return F.batch_norm(y, torch.zeros(c, dtype=torch.float64),
                            torch.ones(c, dtype=torch.float64), tg, tbe, True, 0.1, 1e-5)

    ta = tblock(tx, tw, tb, 0, 1).relu()
    tb2 = tblock(ta, tw, tb, 0, 1).relu()
    ts = tblock(tb2, tdw, tdb, 1, c) + tb2
    tl = F.cross_entropy(F.avg_pool2d(ts, 2, 2).reshape(n, c * 9),
                         torch.tensor(targets, dtype=torch.long))
    tl.backward()
    assert abs(float(prog.value(loss).host()[0]) - tl.item()) <= 1e-5 * abs(tl.item())
    for got, ref, what in ((x, tx, "dx"), (weight.tensor(), tw, "dweight"),
                           (dweight.tensor(), tdw, "dw dweight"), (gamma.tensor(), tg, "dgamma"),
                           (beta.tensor(), tbe, "dbeta")):
        ref = ref.grad.numpy()
        np.testing.assert_allclose(prog.gradient(got).host(), ref, rtol=1e-4,
                                   atol=1e-5 * np.abs(ref).max() + 1e-7, err_msg=what)
    # a bias feeding a training-mode BatchNorm has gradient 0 in exact arithmetic: within the
    # conditioning bound of its sums, 1e-5 * sum|terms| over every use
    terms = [np.abs(y.grad.numpy()).sum(axis=(0, 2, 3)) for y in conv_out]
    for got, ref, bound, what in ((bias.tensor(), tb, terms[0] + terms[1], "dbias"),
                                  (dbias.tensor(), tdb, terms[2], "dw dbias")):
        err = np.abs(prog.gradient(got).host() - ref.grad.numpy())
        assert (err <= 1e-5 * bound + 1e-7).all(), (what, err, bound)



@pytest.mark.parametrize("shortcut", ["relu", "projection"])
def test_batch_norm_add_with_shortcut_built_after_it(shortcut):
    """A training BatchNorm whose only consumer is a residual add, as the add's first operand,
    runs with the add as one launch that writes BN(x) + addend.  Here the addend is created
    after the BatchNorm: relu(x), or a 1x1 convolution + BatchNorm projection of x.  The fused
    launch must run where the addend has been written.  Two runs on different inputs; every
    launch against the oracle, and the loss, the sum and the gradients against torch float64
    autograd each time (the arena starts zero-filled, so an addend read too early shows as
    zeros in the first run and as the previous run's values in the second)."""
    r = np.random.default_rng(53)
    n, c, h, w = 4, 6, 5, 5
    wv = (r.standard_normal((c, c, 3, 3)) * 0.3).astype(np.float32)
    pv = (r.standard_normal((c, c, 1, 1)) * 0.5).astype(np.float32)
    gam, gam2 = r.uniform(0.5, 1.5, c).astype(np.float32), r.uniform(0.5, 1.5, c).astype(np.float32)
    bet, bet2 = r.uniform(-0.2, 0.2, c).astype(np.float32), r.uniform(-0.2, 0.2, c).astype(np.float32)
    zero = np.zeros(c, np.float32)

    x = tn.input((n, c, h, w), requires_grad=True)
    weight, proj = nn.Parameter(wv), nn.Parameter(pv)
    gamma, beta, gamma2, beta2 = (nn.Parameter(v) for v in (gam, bet, gam2, bet2))
    main = x.conv2d(weight.tensor(), tn.constant(zero), 1, 1, 1).batch_norm2d(
        gamma.tensor(), beta.tensor(), tn.BatchNormState(c), True, 0.1, 1e-5)
    if shortcut == "relu":
        skip = x.relu()
    else:
        skip = x.conv2d(proj.tensor(), tn.constant(zero), 1, 0, 1).batch_norm2d(
            gamma2.tensor(), beta2.tensor(), tn.BatchNormState(c), True, 0.1, 1e-5)
    s = main.add(skip)
    t = tn.input((n,))
    loss = s.avg_pool2d((h, w), (h, w)).reshape((n, c)).cross_entropy(t)
    prog = tn.training_program(loss)
    assert [o.kind for o in prog.ops].count("batch_norm2d_add_forward") == 1

    F = torch.nn.functional
    d = lambda v: torch.tensor(v, dtype=torch.float64, requires_grad=True)  # noqa: E731
    for run in range(2):
        xv = r.standard_normal((n, c, h, w)).astype(np.float32)
        targets = r.integers(0, c, n).astype(np.float32)
        prog.feed(x, xv)
        prog.feed(t, targets)
        counts = _run_checked(prog)
        assert counts["batch_norm2d_add_forward"] == 1, dict(counts)
        tx, tw, tp, tg, tb, tg2, tb2 = (d(v) for v in (xv, wv, pv, gam, bet, gam2, bet2))
        stats = lambda: (torch.zeros(c, dtype=torch.float64),  # noqa: E731
                         torch.ones(c, dtype=torch.float64))
        tmain = F.batch_norm(F.conv2d(tx, tw, None, 1, 1), *stats(), tg, tb, True, 0.1, 1e-5)
        tskip = (tx.relu() if shortcut == "relu" else
                 F.batch_norm(F.conv2d(tx, tp), *stats(), tg2, tb2, True, 0.1, 1e-5))
        ts = tmain + tskip
        tl = F.cross_entropy(F.avg_pool2d(ts, (h, w)).reshape(n, c),
                             torch.tensor(targets, dtype=torch.long))
        tl.backward()
        got_loss = float(prog.value(loss).host()[0])
        assert abs(got_loss - tl.item()) <= 1e-5 * abs(tl.item()), (run, got_loss, tl.item())
        ref_s = ts.detach().numpy()
        np.testing.assert_allclose(prog.value(s).host(), ref_s, rtol=1e-4,
                                   atol=1e-5 * np.abs(ref_s).max(), err_msg=f"run {run}: sum")
        grads = [(x, tx, "dx"), (weight.tensor(), tw, "dweight"), (gamma.tensor(), tg, "dgamma"),
                 (beta.tensor(), tb, "dbeta")]
        if shortcut == "projection":
            grads += [(proj.tensor(), tp, "dproj"), (gamma2.tensor(), tg2, "dgamma2"),
                      (beta2.tensor(), tb2, "dbeta2")]
        for got, ref, what in grads:
            ref = ref.grad.numpy()
            np.testing.assert_allclose(prog.gradient(got).host(), ref, rtol=1e-4,
                                       atol=1e-5 * np.abs(ref).max() + 1e-7,
                                       err_msg=f"run {run}: {what}")

def _mnist_batch(r, n):
    images = (r.integers(0, 256, (n, 1, 28, 28)) / 255.0).astype(np.float32)
    labels = r.integers(0, 10, n).astype(np.float32)
    return images, labels


def test_mobilenet_through_generic_builder_matches_native_trainer():
    """MobileNetV4-Conv-S assembled from the generic modules (nn.py) and compiled by
    oxh_net_training_program schedules exactly the native trainer's launch list (same kinds,
    names, tensor roles and shapes), and two eager steps plus one graph replay leave loss,
    all 186 parameters and all running statistics bit-identical."""
    batch = 128
    native = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), batch)
    model = nn.MobileNetV4ConvSmall.mnist()
    x, t = tn.input((batch, 1, 28, 28)), tn.input((batch,))
    loss = model(x).cross_entropy(t)
    prog = tn.training_program(loss, nn.AdamW(1e-3, 1e-4))
    assert [(o.kind, o.name) for o in prog.ops] == [(o.kind, o.name) for o in native.ops]
    for a, b in zip(prog.ops, native.ops):
        assert ({k: [v.shape for v in vs] for k, vs in a.by_role.items()} ==
                {k: [v.shape for v in vs] for k, vs in b.by_role.items()}), a.name
        assert a.attrs.keys() == b.attrs.keys(), a.name
    images, labels = _mnist_batch(np.random.default_rng(41), batch)
    native.set_batch(images, labels)
    prog.feed(x, images)
    prog.feed(t, labels)
    native_params = [p.value for p in native.model.parameters()]
    params = model.parameters()
    assert len(params) == len(native_params) == 186

    def compare(when):
        torch.cuda.synchronize()
        assert_bitexact(prog.value(loss).host(), np.float32([native.loss_value()]), when)
        for i, (p, q) in enumerate(zip(params, native_params)):
            assert_bitexact(p.host(), q.host(), f"{when}: parameter {i}")
        for i, (bn, nbn) in enumerate(zip(model.batch_norms(), native.model.batch_norms())):
            assert_bitexact(host(bn.state.running_mean), nbn.device_running_mean.host(),
                            f"{when}: running mean {i}")
            assert_bitexact(host(bn.state.running_variance),
                            nbn.device_running_variance.host(), f"{when}: running var {i}")

    for step in range(2):
        native.run_eager()
        prog.run()
        compare(f"eager step {step}")
    native.capture()
    prog.capture()
    native.replay()
    prog.replay()
    compare("graph replay")
    assert prog.steps() == native.steps_taken() == 3


def test_whole_program_step_equals_group_by_group_step():
    """A training program with AdamW run whole (oxh_program_run, then captured and replayed)
    against the same program's groups launched one by one (oxh_program_run_op), from the same
    parameters: loss, parameters and parameter gradients bit-identical after every step.  The
    whole program moves the chunk sums of the weight gradients of convolutions whose parameters
    feed them alone (here the strided 3x3 convolution: 512 output positions, more than one
    chunk) into the optimizer group; the 1x1 weight the two later convolutions share keeps its
    sums (its second use adds into the first's gradient).  The 3x3 shape's weight-gradient
    workspace is not empty (its partials are chunked)."""
    r = np.random.default_rng(59)
    n, c, h, w, o = 8, 16, 16, 16, 32
    xv = r.standard_normal((n, c, h, w)).astype(np.float32)
    kv = (r.standard_normal((o, c, 3, 3)) * 0.2).astype(np.float32)
    kb = r.standard_normal(o).astype(np.float32) * 0.1
    pv = (r.standard_normal((o, o, 1, 1)) * 0.3).astype(np.float32)
    pbv = r.standard_normal(o).astype(np.float32) * 0.1
    gam, bet = r.uniform(0.5, 1.5, o).astype(np.float32), r.uniform(-0.2, 0.2, o).astype(np.float32)
    targets = r.integers(0, o, n).astype(np.float32)
    assert ox.conv2d_workspace_size(ox.conv2d_shape(n, c, h, w, o, 3, 2, 1, 1)) > 0

    def build():
        x, t = tn.input((n, c, h, w)), tn.input((n,))
        params = [nn.Parameter(v) for v in (kv, kb, pv, pbv, gam, bet)]
        k, b, p, pb, g, be = (q.tensor() for q in params)
        y = x.conv2d(k, b, 2, 1, 1).batch_norm2d(g, be, tn.BatchNormState(o), True, 0.1, 1e-5)
        y = y.relu().conv2d(p, pb, 1, 0, 1).relu().conv2d(p, pb, 1, 0, 1)
        loss = y.avg_pool2d((8, 8), (8, 8)).reshape((n, o)).cross_entropy(t)
        prog = tn.training_program(loss, nn.AdamW(1e-2, 1e-4))
        prog.feed(x, xv)
        prog.feed(t, targets)
        return prog, loss, params

    groups, whole = build(), build()

    def compare(when):
        torch.cuda.synchronize()
        (pa, la, qa), (pb, lb, qb) = groups, whole
        assert_bitexact(pb.value(lb).host(), pa.value(la).host(), f"{when}: loss")
        for i, (u, v) in enumerate(zip(qa, qb)):
            assert_bitexact(v.host(), u.host(), f"{when}: parameter {i}")
            assert_bitexact(pb.gradient(v.tensor()).host(), pa.gradient(u.tensor()).host(),
                            f"{when}: gradient {i}")

    for step in range(2):
        for op in groups[0].ops:
            op.launch()
        whole[0].run()
        compare(f"step {step}")
    whole[0].capture()
    for step in range(2):
        for op in groups[0].ops:
            op.launch()
        whole[0].replay()
        compare(f"replay {step}")
    assert groups[0].steps() == whole[0].steps() == 4


def test_whole_program_sums_more_convolutions_than_one_launch_takes():
    """Eighteen chained 3x3 convolutions, each with parameters of its own and a chunked weight
    gradient (2048 output positions): the optimizer group sums their chunks in more than one
    launch (at most 16 sums per launch, the step counter advanced by the first).  One whole
    program run and one replay against group-by-group steps: loss, parameters and gradients
    bit for bit, and the step counter advanced once per step."""
    r = np.random.default_rng(61)
    n, c, h, w, depth = 8, 8, 16, 16, 18
    xv = r.standard_normal((n, c, h, w)).astype(np.float32)
    ws = [(r.standard_normal((c, c, 3, 3)) * 0.25).astype(np.float32) for _ in range(depth)]
    bs = [(r.standard_normal(c) * 0.1).astype(np.float32) for _ in range(depth)]
    targets = r.integers(0, c, n).astype(np.float32)
    assert ox.conv2d_workspace_size(ox.conv2d_shape(n, c, h, w, c, 3, 1, 1, 1)) > 0

    def build():
        x, t = tn.input((n, c, h, w)), tn.input((n,))
        params = [nn.Parameter(v) for pair in zip(ws, bs) for v in pair]
        y = x
        for i in range(depth):
            y = y.conv2d(params[2 * i].tensor(), params[2 * i + 1].tensor(), 1, 1, 1)
        loss = y.avg_pool2d((h, w), (h, w)).reshape((n, c)).cross_entropy(t)
        prog = tn.training_program(loss, nn.AdamW(1e-3, 1e-4))
        prog.feed(x, xv)
        prog.feed(t, targets)
        return prog, loss, params

    groups, whole = build(), build()

    def compare(when):
        torch.cuda.synchronize()
        (pa, la, qa), (pb, lb, qb) = groups, whole
        assert_bitexact(pb.value(lb).host(), pa.value(la).host(), f"{when}: loss")
        for i, (u, v) in enumerate(zip(qa, qb)):
            assert_bitexact(v.host(), u.host(), f"{when}: parameter {i}")
            assert_bitexact(pb.gradient(v.tensor()).host(), pa.gradient(u.tensor()).host(),
                            f"{when}: gradient {i}")

    for op in groups[0].ops:
        op.launch()
    whole[0].run()
    compare("run")
    whole[0].capture()
    for op in groups[0].ops:
        op.launch()
    whole[0].replay()
    compare("replay")
    assert groups[0].steps() == whole[0].steps() == 2
