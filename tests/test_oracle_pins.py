"""Pins the CPU oracle before it is trusted as the parity checker.

Each check is chosen so that a plausible restatement mistake (a dropped term, a wrong sign or
index, a swapped operand, a wrong exponent) fails it:
  * the reference's own known-answer tests (tests/golden/reference_kats.json, with sources);
  * torch in float64 on the CPU (textbook batch_norm / cross_entropy / AdamW and autograd);
  * closed forms and invariants (zero logits, t=1 AdamW, exact relu/mul/add identities).
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def f32(x):
    return np.asarray(x, dtype=np.float32)


# ----------------------------------------------------------------- reference KATs


def test_kat_lazy_elementwise_graph():
    kat = KATS["lazy_elementwise_graph_evaluates"]
    x = f32(kat["x"])
    out = oracle.relu(oracle.add(x, np.ones_like(x)))
    assert out.tolist() == kat["expected"]


def test_kat_trace_add_relu():
    kat = KATS["trace_caches_and_reuses_a_graph"]
    out = oracle.relu(oracle.add(f32(kat["x"]), f32(kat["bias"])))
    assert out.tolist() == kat["expected"]


def test_kat_cross_entropy_zero_logits():
    kat = KATS["cross_entropy_backpropagates_softmax_gradient"]
    logits = f32(kat["logits"]).reshape(kat["shape"])
    targets = f32(kat["targets"])
    loss = oracle.ce_forward(logits, targets)
    assert abs(loss - kat["expected_loss"]) < kat["loss_abs_tol"]
    grad = oracle.ce_backward(logits, targets, 1.0)
    assert grad.ravel().tolist() == kat["expected_grad"]


def _bn_ce_loss(data, kat):
    x = f32(data).reshape(kat["shape"])
    y, *_ = oracle.bn_forward(x, f32(kat["weight"]), f32(kat["bias"]), f32(kat["running_mean"]),
                              f32(kat["running_var"]), True, kat["momentum"], kat["epsilon"])
    return oracle.ce_forward(y.reshape(kat["reshape"]), f32(kat["targets"]))


def test_kat_batch_norm_finite_difference():
    kat = KATS["batch_norm_input_gradient_matches_finite_difference"]
    x = f32(kat["input"]).reshape(kat["shape"])
    w, b = f32(kat["weight"]), f32(kat["bias"])
    y, mean, inv_std, _, _ = oracle.bn_forward(x, w, b, f32(kat["running_mean"]),
                                               f32(kat["running_var"]), True, kat["momentum"],
                                               kat["epsilon"])
    g = oracle.ce_backward(y.reshape(kat["reshape"]), f32(kat["targets"]), 1.0)
    dx, dw, db = oracle.bn_backward(g.reshape(x.shape), x, w, mean, inv_std, True)
    step = np.float32(kat["fd_step"])
    for i in range(x.size):
        pos = f32(kat["input"]).copy()
        pos[i] += step
        neg = f32(kat["input"]).copy()
        neg[i] -= step
        numerical = (np.float32(_bn_ce_loss(pos, kat)) - np.float32(_bn_ce_loss(neg, kat))) / (
            np.float32(2.0) * step)
        assert abs(dx.ravel()[i] - numerical) < kat["fd_abs_tol"], (i, dx.ravel()[i], numerical)
    assert dw.shape == (2,) and db.shape == (2,)


def test_kat_batch_norm_running_stats_and_eval():
    kat = KATS["batch_norm_updates_running_statistics_and_switches_to_eval"]
    x = f32(kat["input"]).reshape(kat["shape"])
    c = kat["channels"]
    w, b = np.ones(c, np.float32), np.zeros(c, np.float32)
    y, _, _, rm, rv = oracle.bn_forward(x, w, b, np.zeros(c, np.float32), np.ones(c, np.float32))
    for ch in range(c):
        assert abs(float(y[:, ch].mean())) < kat["output_channel_mean_abs_tol"]
    assert np.all(np.abs(rm - f32(kat["expected_running_mean"])) < kat["running_mean_abs_tol"])
    assert rv[0] > kat["running_var0_greater_than"]
    y_eval, *_ = oracle.bn_forward(x, w, b, rm, rv, training=False)
    assert not np.array_equal(y, y_eval)


def test_kat_traced_batch_norm_recomputes_stats():
    kat = KATS["traced_batch_norm_recomputes_batch_statistics_each_run"]
    rm, rv = np.zeros(1, np.float32), np.ones(1, np.float32)
    for run in kat["runs"]:
        x = f32(run).reshape(kat["shape"])
        y, _, _, rm, rv = oracle.bn_forward(x, np.ones(1, np.float32), np.zeros(1, np.float32),
                                            rm, rv)
        assert np.all(np.abs(y.ravel() - f32(kat["expected"])) < kat["abs_tol"])


def test_kat_adamw_reduces_loss():
    """optim.rs:168-208 with the 1x1 conv harness written out in numpy (conv is not on the path)."""
    kat = KATS["adamw_reduces_a_tiny_classification_loss"]
    x = f32(kat["input"])
    targets = f32(kat["targets"])
    weight = oracle.initialized_weights([2, 1, 1, 1], 1).ravel().copy()
    bias = np.zeros(2, np.float32)

    def logits_of(w, b):
        return (x[:, None] * w[None, :] + b[None, :]).astype(np.float32)

    initial = oracle.ce_forward(logits_of(weight, bias), targets)
    mw, vw = np.zeros(2, np.float32), np.zeros(2, np.float32)
    mb, vb = np.zeros(2, np.float32), np.zeros(2, np.float32)
    for step in range(1, kat["steps"] + 1):
        g = oracle.ce_backward(logits_of(weight, bias), targets, 1.0)
        gw = (g * x[:, None]).sum(axis=0).astype(np.float32)
        gb = g.sum(axis=0).astype(np.float32)
        weight, mw, vw = oracle.adamw_update(weight, gw, mw, vw, step, lr=kat["learning_rate"],
                                             weight_decay=kat["weight_decay"])
        bias, mb, vb = oracle.adamw_update(bias, gb, mb, vb, step, lr=kat["learning_rate"],
                                           weight_decay=kat["weight_decay"])
    final = oracle.ce_forward(logits_of(weight, bias), targets)
    assert final < initial


# ----------------------------------------------------------------- elementwise identities


def test_elementwise_exact(rng):
    a = rng.uniform(-1, 1, 4099).astype(np.float32)
    b = rng.uniform(-1, 1, 4099).astype(np.float32)
    c = rng.uniform(-1, 1, 4099).astype(np.float32)
    assert np.array_equal(oracle.add(a, b), a + b)
    assert np.array_equal(oracle.mul(a, b), a * b)
    assert np.array_equal(oracle.relu(a), np.where(a > 0, a, np.float32(0)))
    assert np.array_equal(oracle.relu_backward(b, a), np.where(a > 0, b, np.float32(0)))
    assert np.array_equal(oracle.mul_backward(b, c), b * c)
    assert np.array_equal(oracle.accumulate(a, b), a + b)
    s = a + b
    m = s * c
    assert np.array_equal(oracle.chain_forward(a, b, c), np.maximum(m, np.float32(0)))
    da, db, dc = oracle.chain_backward_ones(a, b, c)
    on = m > 0
    assert np.array_equal(da, np.where(on, c, np.float32(0)))
    assert np.array_equal(db, da)
    assert np.array_equal(dc, np.where(on, s, np.float32(0)))


def test_relu_nan_and_signed_zero():
    x = f32([np.nan, -0.0, 0.0, -np.inf, np.inf])
    out = oracle.relu(x)
    assert out[0] == 0.0 and out[1] == 0.0 and out[2] == 0.0 and out[3] == 0.0
    assert out[4] == np.inf


# ----------------------------------------------------------------- torch float64 cross-checks

torch = pytest.importorskip("torch")


def _bn_torch64(x, w, b, rm, rv, g, training, momentum=0.1, eps=1e-5):
    x64 = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    w64 = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    b64 = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    rm64 = torch.tensor(rm, dtype=torch.float64)
    rv64 = torch.tensor(rv, dtype=torch.float64)
    y = torch.nn.functional.batch_norm(x64, rm64, rv64, w64, b64, training=training,
                                       momentum=momentum, eps=eps)
    y.backward(torch.tensor(g, dtype=torch.float64))
    return (y.detach().numpy(), rm64.numpy(), rv64.numpy(), x64.grad.numpy(), w64.grad.numpy(),
            b64.grad.numpy())


@pytest.mark.parametrize("shape", [(2, 3, 4, 5), (5, 4, 7, 7), (3, 2, 1, 1), (1, 3, 1, 9)])
@pytest.mark.parametrize("training", [True, False])
def test_batch_norm_matches_torch_float64(rng, shape, training):
    n, c, h, w = shape
    x = (rng.standard_normal(shape) * 1.7 + 0.3).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, c).astype(np.float32)
    beta = rng.uniform(-0.1, 0.1, c).astype(np.float32)
    rm = rng.uniform(-0.5, 0.5, c).astype(np.float32)
    rv = rng.uniform(0.5, 2.0, c).astype(np.float32)
    g = rng.standard_normal(shape).astype(np.float32)
    y, mean, inv_std, rm1, rv1 = oracle.bn_forward(x, gamma, beta, rm, rv, training)
    dx, dw, db = oracle.bn_backward(g, x, gamma, mean, inv_std, training)
    ty, trm, trv, tdx, tdw, tdb = _bn_torch64(x, gamma, beta, rm, rv, g, training)
    np.testing.assert_allclose(y, ty, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(rm1, trm, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rv1, trv, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(dx, tdx, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dw, tdw, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(db, tdb, rtol=1e-4, atol=1e-5)


def test_batch_norm_training_invariants(rng):
    x = rng.standard_normal((4, 3, 5, 5)).astype(np.float32)
    g = rng.standard_normal(x.shape).astype(np.float32)
    gamma = rng.uniform(0.5, 1.5, 3).astype(np.float32)
    beta = rng.uniform(-0.1, 0.1, 3).astype(np.float32)
    y, mean, inv_std, _, _ = oracle.bn_forward(x, gamma, beta, np.zeros(3, np.float32),
                                               np.ones(3, np.float32))
    x64 = x.astype(np.float64)
    np.testing.assert_allclose(mean, x64.mean(axis=(0, 2, 3)), atol=1e-6)
    np.testing.assert_allclose(inv_std, 1 / np.sqrt(x64.var(axis=(0, 2, 3)) + 1e-5), rtol=1e-5)
    np.testing.assert_allclose(y.astype(np.float64).mean(axis=(0, 2, 3)), beta, atol=1e-5)
    dx, dw, db = oracle.bn_backward(g, x, gamma, mean, inv_std, True)
    # training-mode input gradient is orthogonal to 1 and to x_hat per channel
    xhat = (x64 - mean[None, :, None, None]) * inv_std[None, :, None, None]
    # exact-arithmetic identities: tolerance scales with the sum of |terms| (fp32 rounding)
    scale_1 = np.abs(dx).astype(np.float64).sum(axis=(0, 2, 3))
    scale_x = np.abs(dx * xhat).sum(axis=(0, 2, 3))
    assert np.all(np.abs(dx.astype(np.float64).sum(axis=(0, 2, 3))) <= 1e-5 * scale_1)
    assert np.all(np.abs((dx * xhat).sum(axis=(0, 2, 3))) <= 1e-5 * scale_x)
    np.testing.assert_allclose(db, g.astype(np.float64).sum(axis=(0, 2, 3)), rtol=1e-5, atol=1e-5)


def test_batch_norm_rejects_single_sample():
    x = np.ones((1, 2, 1, 1), np.float32)
    with pytest.raises(oracle.OracleError) as err:
        oracle.bn_forward(x, np.ones(2, np.float32), np.zeros(2, np.float32),
                          np.zeros(2, np.float32), np.ones(2, np.float32))
    assert err.value.kind == "Execution"


@pytest.mark.parametrize("shape", [(4, 7), (3, 1000), (2, 1)])
def test_cross_entropy_matches_torch_float64(rng, shape):
    b, k = shape
    logits = (rng.standard_normal(shape) * 2).astype(np.float32)
    targets = rng.integers(0, k, b).astype(np.float32)
    outer = 0.75
    loss = oracle.ce_forward(logits, targets)
    grad = oracle.ce_backward(logits, targets, outer)
    t = torch.tensor(logits, dtype=torch.float64, requires_grad=True)
    tl = torch.nn.functional.cross_entropy(t, torch.tensor(targets.astype(np.int64)))
    (tl * outer).backward()
    assert abs(loss - tl.item()) <= 1e-5 * abs(tl.item()) + 1e-6
    np.testing.assert_allclose(grad, t.grad.numpy(), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(grad.astype(np.float64).sum(axis=1), 0, atol=1e-6)


def test_cross_entropy_zero_logits_closed_form():
    b, k = 3, 5
    logits = np.zeros((b, k), np.float32)
    targets = f32([0, 4, 2])
    assert abs(oracle.ce_forward(logits, targets) - math.log(k)) < 1e-6
    grad = oracle.ce_backward(logits, targets, 1.0)
    expect = np.full((b, k), (1 / k) / b)
    expect[np.arange(b), targets.astype(int)] -= 1 / b
    np.testing.assert_allclose(grad, expect, rtol=1e-6, atol=1e-8)


@pytest.mark.parametrize("value,ok", [(3.0, True), (0.0, True), (-0.0, True), (1.5, False),
                                      (-1.0, False), (float("nan"), False), (float("inf"), False),
                                      (5.0, False), (1e30, False), (2.0 ** 64, False),
                                      (2.0 ** 63, False)])
def test_class_index_rules(value, ok):
    if ok:
        assert oracle.class_index(value, 5) == int(abs(value))
    else:
        with pytest.raises(oracle.OracleError) as err:
            oracle.class_index(value, 5)
        assert err.value.kind == "InvalidShape"


def test_powi_binary_exponentiation():
    assert oracle.powi(2.0, 10) == 1024.0
    assert oracle.powi(0.5, -3) == 8.0
    assert oracle.powi(3.0, 0) == 1.0
    for base in (0.9, 0.999, 1.7):
        for e in (1, 2, 3, 10, 17, -2):
            assert abs(oracle.powi(base, e) - base ** e) <= 4e-7 * abs(base ** e) * abs(e), (base, e)
    # powi(-2) of the epsilon-free inverse std returns the biased variance
    v = np.float32(0.3)
    inv = np.float32(1.0) / np.sqrt(v)
    assert abs(oracle.powi(float(inv), -2) - 0.3) < 1e-7


def _torch_adamw(p, g_list, m0, v0, step0, lr, wd):
    t = torch.tensor(p, dtype=torch.float64, requires_grad=True)
    # the reference holds its hyper-parameters as f32 (optim.rs:35-46): give torch those values
    r = lambda v: float(np.float32(v))  # noqa: E731
    opt = torch.optim.AdamW([t], lr=r(lr), betas=(r(0.9), r(0.999)), eps=r(1e-8),
                            weight_decay=r(wd))
    opt.state[t] = {"step": torch.tensor(float(step0), dtype=torch.float64),
                    "exp_avg": torch.tensor(m0, dtype=torch.float64),
                    "exp_avg_sq": torch.tensor(v0, dtype=torch.float64)}
    for g in g_list:
        t.grad = torch.tensor(g, dtype=torch.float64)
        opt.step()
    st = opt.state[t]
    return t.detach().numpy(), st["exp_avg"].numpy(), st["exp_avg_sq"].numpy()


def test_adamw_matches_torch_float64(rng):
    n = 2048
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    m0 = (0.1 * rng.standard_normal(n) * 1e-3).astype(np.float32)
    v0 = (0.001 * (rng.standard_normal(n) * 1e-3) ** 2).astype(np.float32)
    grads = [(rng.standard_normal(n) * 1e-3).astype(np.float32) for _ in range(3)]
    pp, mm, vv = p, m0, v0
    for i, g in enumerate(grads):
        pp, mm, vv = oracle.adamw_update(pp, g, mm, vv, 10 + i, lr=1e-3, weight_decay=0.01)
    tp, tm, tv = _torch_adamw(p, grads, m0, v0, 9, 1e-3, 0.01)
    # bound by the magnitude of the summed terms (m and v cancel near zero)
    m_terms = np.abs(m0).astype(np.float64) + sum(np.abs(g).astype(np.float64) for g in grads)
    np.testing.assert_allclose(vv, tv, rtol=1e-5, atol=1e-15)
    assert np.all(np.abs(mm - tm) <= 1e-5 * m_terms)
    assert np.all(np.abs(pp - tp) <= 1e-5 * np.abs(tp) + 1e-5 * 1e-3 * len(grads))


def test_adamw_first_step_closed_form(rng):
    p = rng.standard_normal(512).astype(np.float32)
    g = rng.standard_normal(512).astype(np.float32)
    z = np.zeros_like(p)
    lr, wd = 1e-2, 0.1
    new_p, m, v = oracle.adamw_update(p, g, z, z, 1, lr=lr, weight_decay=wd)
    expect = p.astype(np.float64) - lr * (np.sign(g) + wd * p.astype(np.float64))
    np.testing.assert_allclose(new_p, expect, rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------------- argmax / init


def test_argmax_last_index_wins_ties():
    rows = f32([[1, 3, 3, 2], [0, -0.0, 0.0, -1], [5, 5, 5, 5], [np.nan, 1, 2, 3],
                [-np.inf, -np.inf, -np.inf, -np.inf]])
    assert oracle.argmax_rows(rows).tolist() == [2, 2, 3, 0, 3]


def test_initialized_weights_properties():
    w1 = oracle.initialized_weights([8, 4, 3, 3], 4)
    w2 = oracle.initialized_weights([8, 4, 3, 3], 4)
    assert np.array_equal(w1, w2)
    scale = math.sqrt(2.0 / 36)
    assert np.all(np.abs(w1) <= scale)
    assert abs(float(w1.mean())) < 0.1 * scale
    assert not np.array_equal(w1, oracle.initialized_weights([4, 8, 3, 3], 8).reshape(w1.shape))
