"""Config 5: the MobileNetV4-Conv-S MNIST training step (examples/mnist_training.rs:75-92)
through liboxide_hip.so, every scheduled launch recomputed by the oracle from the device
inputs it actually read.

Per-op bars: conv forward / input gradient, pooling, ReLU, add, accumulate, argmax and AdamW
bit-exact; BatchNorm and cross entropy within the north star's 1e-5 relative (1e-6 absolute,
or the conditioning bound of a cancelling sum); conv weight / bias gradients within
1e-5 * sum|terms| (fixed-order chunked sums)."""

from collections import Counter

import numpy as np
import pytest
import torch

import oracle
import oxide_hip as ox
import training as T
from helpers import (assert_bitexact, assert_close, assert_within, check_batch_norm_backward,
                     check_batch_norm_forward, host)

pytestmark = pytest.mark.gpu


def _mnist_batch(r, n):
    """Synthetic MNIST-shaped batch: pixels k / 255, labels uniform over the 10 classes."""
    images = (r.integers(0, 256, (n, 1, 28, 28)) / 255.0).astype(np.float32)
    labels = r.integers(0, 10, n).astype(np.float32)
    return images, labels


class OracleChecker:
    """``before`` snapshots what an op updates in place; ``after`` recomputes the op with the
    oracle from the device tensors it read and compares what it wrote."""

    def __init__(self):
        self.prior = {}
        self.counts = Counter()

    def before(self, op):
        torch.cuda.synchronize()
        self.prior = {id(t): host(t).copy() for t in op.inplace}

    def after(self, op):
        torch.cuda.synchronize()
        getattr(self, op.kind)(op, {k: host(v) for k, v in op.reads.items()})
        if op.accumulate_into is not None:
            prev = self.prior[id(op.accumulate_into)]
            assert_bitexact(host(op.accumulate_into),
                            oracle.accumulate(prev, host(op.writes["contribution"])),
                            f"{op.name} accumulate")
        self.counts[op.kind] += 1

    # -- per kind
    def conv2d_forward(self, op, r):
        a = op.attrs
        ref = oracle.conv2d_forward(r["x"], r["weight"], r["bias"], a["stride"], a["padding"],
                                    a["groups"])
        assert_bitexact(host(op.writes["y"]), ref, op.name)

    def conv2d_input_backward(self, op, r):
        a = op.attrs
        ref = oracle.conv2d_backward(r["gradient"], r["x"], r["weight"], a["stride"],
                                     a["padding"], a["groups"])[0]
        if "addend" in r:  # a residual add's gradient accumulated in the same pass
            ref = oracle.accumulate(r["addend"], ref)
            self.counts["conv input backward with addend"] += 1
        assert_bitexact(host(op.writes["contribution"]), ref, op.name)

    def conv2d_parameter_backward(self, op, r):
        a = op.attrs
        g, x, w = r["gradient"], r["x"], r["weight"]
        _, rdw, rdb = oracle.conv2d_backward(g, x, w, a["stride"], a["padding"], a["groups"])
        abs_dw = oracle.conv2d_backward(np.abs(g), np.abs(x), np.abs(w), a["stride"],
                                        a["padding"], a["groups"])[1]
        assert_within(host(op.writes["weight_gradient"]), rdw,
                      1e-5 * abs_dw.astype(np.float64) + 1e-7, f"{op.name} weight")
        if "bias_gradient" in op.writes:  # else the following BatchNorm's backward formed it
            assert_within(host(op.writes["bias_gradient"]), rdb,
                          1e-5 * np.abs(g).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                          f"{op.name} bias")
            self.counts["conv bias in parameter backward"] += 1

    def _conv_bias(self, op):
        """The bias gradient of the convolution feeding a BatchNorm, formed by the BN backward
        from the input gradient it wrote."""
        if "conv_bias_gradient" not in op.writes:
            return
        dx = host(op.writes["contribution"])
        assert_within(host(op.writes["conv_bias_gradient"]), oracle.conv2d_bias_backward(dx),
                      1e-5 * np.abs(dx).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                      f"{op.name} conv bias")
        self.counts["conv bias in batch norm backward"] += 1

    def batch_norm2d_forward(self, op, r):
        a, w = op.attrs, op.writes
        out = dict(y=host(w["y"]), mean=host(w["saved_mean"]), inv=host(w["saved_inverse_std"]),
                   rm=host(a["running_mean"]), rv=host(a["running_variance"]))
        check_batch_norm_forward(out, r["x"], r["weight"], r["bias"],
                                 self.prior[id(a["running_mean"])],
                                 self.prior[id(a["running_variance"])], a["momentum"],
                                 a["epsilon"])

    def batch_norm2d_add_forward(self, op, r):
        """BN forward writing BN(x) + shortcut: the statistics against the oracle, the output
        equal to the fp32 normalization with those statistics followed by the add."""
        a, w = op.attrs, op.writes
        x, gamma, beta = r["x"], r["weight"], r["bias"]
        mean, inv = host(w["saved_mean"]), host(w["saved_inverse_std"])
        sh = (1, x.shape[1], 1, 1)
        y_bn = ((x - mean.reshape(sh)) * inv.reshape(sh)) * gamma.reshape(sh) + beta.reshape(sh)
        out = dict(y=y_bn, mean=mean, inv=inv, rm=host(a["running_mean"]),
                   rv=host(a["running_variance"]))
        check_batch_norm_forward(out, x, gamma, beta, self.prior[id(a["running_mean"])],
                                 self.prior[id(a["running_variance"])], a["momentum"],
                                 a["epsilon"])
        assert_bitexact(host(w["y"]), oracle.add(y_bn, r["addend"]), op.name)

    def batch_norm2d_backward(self, op, r):
        w = op.writes
        out = dict(dx=host(w["contribution"]), dw=host(w["weight_gradient"]),
                   db=host(w["bias_gradient"]))
        check_batch_norm_backward(out, r["gradient"], r["x"], r["weight"], r["saved_mean"],
                                  r["saved_inverse_std"])
        self._conv_bias(op)

    def batch_norm2d_relu_forward(self, op, r):
        a, w = op.attrs, op.writes
        out = dict(y=host(w["y"]), mean=host(w["saved_mean"]), inv=host(w["saved_inverse_std"]),
                   rm=host(a["running_mean"]), rv=host(a["running_variance"]))
        assert (out["y"] >= 0).all()
        check_batch_norm_forward(out, r["x"], r["weight"], r["bias"],
                                 self.prior[id(a["running_mean"])],
                                 self.prior[id(a["running_variance"])], a["momentum"],
                                 a["epsilon"], relu=True)

    def batch_norm2d_relu_backward(self, op, r):
        w = op.writes
        out = dict(dx=host(w["contribution"]), dw=host(w["weight_gradient"]),
                   db=host(w["bias_gradient"]))
        masked = oracle.relu_backward(r["gradient"], r["y"])
        check_batch_norm_backward(out, masked, r["x"], r["weight"], r["saved_mean"],
                                  r["saved_inverse_std"])
        self._conv_bias(op)

    def _depthwise_forward(self, op, r, relu):
        """Depthwise conv + BN (+ ReLU) in one launch: the convolution output bit-exact, the
        BatchNorm on it as a separate BatchNorm forward is checked."""
        a, w = op.attrs, op.writes
        conv_y = host(w["conv_y"])
        assert_bitexact(conv_y, oracle.conv2d_forward(r["x"], r["conv_weight"], r["conv_bias"],
                                                      a["stride"], a["padding"], a["groups"]),
                        f"{op.name} conv")
        out = dict(y=host(w["y"]), mean=host(w["saved_mean"]), inv=host(w["saved_inverse_std"]),
                   rm=host(a["running_mean"]), rv=host(a["running_variance"]))
        check_batch_norm_forward(out, conv_y, r["weight"], r["bias"],
                                 self.prior[id(a["running_mean"])],
                                 self.prior[id(a["running_variance"])], a["momentum"],
                                 a["epsilon"], relu=relu)

    def depthwise_conv2d_batch_norm_forward(self, op, r):
        self._depthwise_forward(op, r, False)

    def depthwise_conv2d_batch_norm_relu_forward(self, op, r):
        self._depthwise_forward(op, r, True)

    def _depthwise_backward(self, op, r, relu):
        """Its backward: the BatchNorm gradients as a BatchNorm backward's, then the
        convolution's bias / weight gradients (fixed-order sums) and input gradient (bit-exact,
        + the residual addend where one is folded in) from the output gradient it wrote."""
        a, w = op.attrs, op.writes
        gc = host(w["conv_output_gradient"])
        g = oracle.relu_backward(r["gradient"], r["y"]) if relu else r["gradient"]
        check_batch_norm_backward(dict(dx=gc, dw=host(w["weight_gradient"]),
                                       db=host(w["bias_gradient"])), g, r["conv_y"],
                                  r["weight"], r["saved_mean"], r["saved_inverse_std"])
        x, cw = r["x"], r["conv_weight"]
        s, p, grp = a["stride"], a["padding"], a["groups"]
        rdx, rdw, rdb = oracle.conv2d_backward(gc, x, cw, s, p, grp)
        abs_dw = oracle.conv2d_backward(np.abs(gc), np.abs(x), np.abs(cw), s, p, grp)[1]
        assert_within(host(w["conv_weight_gradient"]), rdw,
                      1e-5 * abs_dw.astype(np.float64) + 1e-7, f"{op.name} conv weight")
        assert_within(host(w["conv_bias_gradient"]), rdb,
                      1e-5 * np.abs(gc).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                      f"{op.name} conv bias")
        self.counts["conv bias in batch norm backward"] += 1
        if "contribution" in w:
            if "addend" in r:
                rdx = oracle.accumulate(r["addend"], rdx)
                self.counts["conv input backward with addend"] += 1
            assert_bitexact(host(w["contribution"]), rdx, f"{op.name} input gradient")

    def depthwise_conv2d_batch_norm_backward(self, op, r):
        self._depthwise_backward(op, r, False)

    def depthwise_conv2d_batch_norm_relu_backward(self, op, r):
        self._depthwise_backward(op, r, True)

    def relu_forward(self, op, r):
        assert_bitexact(host(op.writes["y"]), oracle.relu(r["x"]), op.name)

    def relu_backward(self, op, r):
        assert_bitexact(host(op.writes["contribution"]),
                        oracle.relu_backward(r["gradient"], r["x"]), op.name)

    def add_forward(self, op, r):
        assert_bitexact(host(op.writes["y"]), oracle.add(r["a"], r["b"]), op.name)

    def add_backward(self, op, r):
        assert_bitexact(host(op.writes["contribution"]), r["gradient"], op.name)

    def avg_pool2d_forward(self, op, r):
        a = op.attrs
        assert_bitexact(host(op.writes["y"]),
                        oracle.avg_pool2d_forward(r["x"], a["kernel"], a["stride"]), op.name)

    def avg_pool2d_backward(self, op, r):
        a = op.attrs
        assert_bitexact(host(op.writes["contribution"]),
                        oracle.avg_pool2d_backward(r["gradient"], op.writes["contribution"].shape,
                                                   a["kernel"], a["stride"]), op.name)

    def cross_entropy(self, op, r):
        logits, targets = r["logits"], r["targets"]
        outer = float(r["outer_gradient"][0])
        assert_close(host(op.writes["loss"]).astype(np.float32),
                     np.float32([oracle.ce_forward(logits, targets)]), what="loss")
        assert_close(host(op.writes["gradient"]), oracle.ce_backward(logits, targets, outer),
                     atol=1e-6 * abs(outer) / logits.shape[0], what="logit gradient")
        assert int(host(op.inplace[0])[0]) == 0

    def adamw(self, op, r):
        a = op.attrs
        step = int(host(a["step_counter"])[0])
        assert step == int(self.prior[id(a["step_counter"])][0]) + 1
        for i, (p, g, m, v) in enumerate(a["tensors"]):
            rp, rm, rv = oracle.adamw_update(self.prior[id(p)], host(g), self.prior[id(m)],
                                             self.prior[id(v)], step, a["learning_rate"],
                                             a["weight_decay"], a["beta1"], a["beta2"],
                                             a["epsilon"])
            assert_bitexact(host(p), rp, f"adamw parameter {i}")
            assert_bitexact(host(m), rm, f"adamw first moment {i}")
            assert_bitexact(host(v), rv, f"adamw second moment {i}")


# 46 BatchNorms, 32 of them followed by a ReLU (fused), each fed by a convolution whose bias
# gradient its backward forms (the classifier's, fed by no BN, stays with its parameter
# backward); the 15 depthwise convolutions run with their BatchNorm + ReLU in one launch per
# direction; 10 residual adds, formed by the forward of the BN feeding them, whose first
# operand's gradient is the add's own buffer and whose second operand's is added by that
# operand's convolution input backward (no add launches in either direction)
EXPECTED_KINDS = {"conv2d_forward": 32, "conv2d_parameter_backward": 32,
                  "conv2d_input_backward": 31, "batch_norm2d_forward": 4,
                  "batch_norm2d_add_forward": 10,
                  "batch_norm2d_relu_forward": 17, "batch_norm2d_backward": 14,
                  "batch_norm2d_relu_backward": 17,
                  "depthwise_conv2d_batch_norm_relu_forward": 15,
                  "depthwise_conv2d_batch_norm_relu_backward": 15,
                  "conv input backward with addend": 10,
                  "avg_pool2d_forward": 1, "avg_pool2d_backward": 1, "cross_entropy": 1,
                  "adamw": 1, "conv bias in parameter backward": 1,
                  "conv bias in batch norm backward": 46}


def test_config5_step_every_op_matches_oracle():
    """Two eager steps at batch 128 (the second with non-zero Adam moments and updated BN
    running statistics), every launch checked."""
    step = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), 128)
    r = np.random.default_rng(0x6F78696400000005)
    for i in range(2):
        step.set_batch(*_mnist_batch(r, 128))
        checker = OracleChecker()
        step.run_eager(checker.before, checker.after)
        assert dict(checker.counts) == EXPECTED_KINDS
        assert np.isfinite(step.loss_value())
    assert step.steps_taken() == 2
    # argmax over the device logits (ties to the last index), bit-exact
    classes = step.predicted_classes()
    np.testing.assert_array_equal(classes, oracle.argmax_rows(host(step.logits)))


def test_device_parameters_equal_oracle_init():
    """Every parameter oxh_mnv4_create uploads equals the oracle's nn.rs:657-674 init bit for
    bit (conv weights; zero conv biases, BatchNorm gamma 1 / beta 0 as nn.rs:139-140 and
    271-273), and every running statistic starts at mean 0 / variance 1."""
    model = T.MobileNetV4ConvSmall.mnist()
    params = model.parameters()
    assert len(params) == 186
    kinds = Counter()
    for i, p in enumerate(params):
        got = p.value.host()
        if len(p.shape) == 4:
            ref = oracle.initialized_weights(list(p.shape), p.shape[1]).reshape(p.shape)
            kinds["weight"] += 1
        else:
            # visit order: conv weight, conv bias, then the BatchNorm's gamma and beta
            is_gamma = len(params[i - 1].shape) == 1 and len(params[i - 2].shape) == 4
            ref = np.full(p.shape, 1.0 if is_gamma else 0.0, np.float32)
            kinds["gamma" if is_gamma else "zero"] += 1
        assert_bitexact(got, ref, f"parameter {i} {p.shape}")
    assert kinds == {"weight": 47, "gamma": 46, "zero": 93}
    for bn in model.batch_norms():
        assert_bitexact(bn.device_running_mean.host(), np.zeros(bn.channels, np.float32), "rm")
        assert_bitexact(bn.device_running_variance.host(), np.ones(bn.channels, np.float32), "rv")


def test_reference_full_training_step():
    """mobilenet_v4.rs:468-483: zero images [2, 1, 28, 28], targets [3, 7], one AdamW(1e-3,
    1e-4) step.  With zero input every activation is zero, the logits are zero and the loss is
    ln 10; every op is still checked against the oracle."""
    step = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), 2)
    step.set_batch(np.zeros((2, 1, 28, 28), np.float32), np.array([3.0, 7.0], np.float32))
    checker = OracleChecker()
    step.run_eager(checker.before, checker.after)
    loss = step.loss_value()
    assert np.isfinite(loss) and abs(loss - np.log(10.0)) < 1e-6
    assert dict(checker.counts) == EXPECTED_KINDS


def _state(step):
    torch.cuda.synchronize()
    out = [host(p.value) for p in step.params]
    out += [host(t) for bn in step.model.batch_norms()
            for t in (bn.device_running_mean, bn.device_running_variance)]
    return out


def test_graph_replay_matches_eager_bitwise():
    """The captured step replayed 3 times leaves parameters, moments, running statistics and
    loss bit-identical to 3 eager steps (every kernel sums in a fixed order)."""
    r = np.random.default_rng(17)
    batch = _mnist_batch(r, 128)
    eager = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), 128)
    eager.set_batch(*batch)
    eager_losses = []
    for _ in range(3):
        eager.run_eager()
        eager_losses.append(eager.loss_value())
    graph = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), 128)
    graph.set_batch(*batch)
    graph.capture()
    graph_losses = []
    for _ in range(3):
        graph.replay()
        graph_losses.append(graph.loss_value())
        torch.cuda.synchronize()  # eager work between replays
    assert graph_losses == eager_losses
    assert graph.steps_taken() == 3
    for i, (a, b) in enumerate(zip(_state(eager), _state(graph))):
        assert_bitexact(b, a, f"state tensor {i}")


def test_loss_decreases_on_a_fixed_batch():
    """AdamW(1e-3, 1e-4) on one batch of 128: the loss falls well below its start within 30
    replayed steps."""
    step = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), 128)
    step.set_batch(*_mnist_batch(np.random.default_rng(5), 128))
    step.capture()
    losses = []
    for _ in range(30):
        step.replay()
        losses.append(step.loss_value())
    assert all(np.isfinite(losses))
    assert losses[-1] < 0.5 * losses[0], losses


def test_invalid_target_raises():
    """A label outside [0, 10) raises InvalidShape when the loss is read (the CPU path's
    error, evaluation.rs:622-636); as on the reference's GPU path, the kernels of that step
    have already run with a NaN row."""
    step = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), 4)
    step.set_batch(np.zeros((4, 1, 28, 28), np.float32), np.array([0, 1, 10, 2], np.float32))
    step.run_eager()
    with pytest.raises(ox.OxideError) as e:
        step.loss_value()
    assert e.value.status == ox.INVALID_SHAPE
