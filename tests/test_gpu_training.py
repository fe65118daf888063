"""Config 5: the MobileNetV4-Conv-S MNIST training step (examples/mnist_training.rs:75-92)
through liboxide_hip.so, every scheduled launch recomputed by the oracle from the device
inputs it actually read.

Per-op bars: the conv input gradients and forwards the library sums in the CPU path's order
(oxh_conv2d_input_backward_serial, oxh_conv2d_forward_serial), pooling, ReLU, add,
accumulate, argmax and AdamW bit-exact; BatchNorm and cross entropy within the north star's
1e-5 relative (1e-6 absolute, or the conditioning bound of a cancelling sum); the other conv
input gradients and forwards and conv weight / bias gradients within 1e-5 * sum|terms|
(fixed-order sums over contiguous parts)."""

from collections import Counter

import numpy as np
import pytest
import torch

import oracle
import oxide_hip as ox
import training as T
from helpers import assert_bitexact, host
from oracle_checker import OracleChecker

pytestmark = pytest.mark.gpu


def _mnist_batch(r, n):
    """Synthetic MNIST-shaped batch: pixels k / 255, labels uniform over the 10 classes."""
    images = (r.integers(0, 256, (n, 1, 28, 28)) / 255.0).astype(np.float32)
    labels = r.integers(0, 10, n).astype(np.float32)
    return images, labels


# Every convolution but the stem (whose input, the image, takes no gradient) forms its weight
# and input gradients in one launch group.
# The BatchNorm in front of each of the 15 depthwise layers runs inside that layer's launches:
# the 11 UIB expand BatchNorms (+ ReLU) before the middle depthwise layers, and before the 4
# start depthwise layers the previous block's last BatchNorm (2 with the residual add).
# 46 BatchNorms, 32 of them followed by a ReLU (fused), each fed by a convolution whose bias
# gradient its backward forms, but for the stem's (its 14x14 BatchNorm is no one-block-per-
# channel kernel: the stem's parameter backward sums the bias with its weight gradient) and the
# classifier's (fed by no BN); the 15 depthwise convolutions run with their BatchNorm + ReLU in one launch per
# direction; 10 residual adds, formed by the forward of the BN feeding them, whose first
# operand's gradient is the add's own buffer and whose second operand's is added by that
# operand's convolution input backward (no add launches in either direction)
EXPECTED_KINDS = {"conv2d_forward": 32, "conv2d_parameter_backward": 1,
                  "conv2d_backward": 31, "batch_norm2d_forward": 2,
                  "batch_norm2d_add_forward": 8,
                  "batch_norm2d_relu_forward": 6, "batch_norm2d_backward": 10,
                  "batch_norm2d_relu_backward": 6,
                  "batch_norm2d_relu_depthwise_conv2d_batch_norm_relu_forward": 11,
                  "batch_norm2d_relu_depthwise_conv2d_batch_norm_relu_backward": 11,
                  "batch_norm2d_depthwise_conv2d_batch_norm_relu_forward": 2,
                  "batch_norm2d_depthwise_conv2d_batch_norm_relu_backward": 2,
                  "batch_norm2d_add_depthwise_conv2d_batch_norm_relu_forward": 2,
                  "batch_norm2d_add_depthwise_conv2d_batch_norm_relu_backward": 2,
                  "batch norm before depthwise": 30,
                  "conv input backward with addend": 10,
                  "cross_entropy": 1,
                  "adamw": 1, "conv bias in parameter backward": 2,
                  "conv bias in batch norm backward": 45}


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
    loss bit-identical to 3 eager steps launched group by group (every kernel sums in a fixed
    order).  Group by group, each convolution sums its own weight-gradient chunks; the whole
    program (run or captured) sums them all in one launch before AdamW: the same values."""
    r = np.random.default_rng(17)
    batch = _mnist_batch(r, 128)
    eager = T.TrainingStep(T.MobileNetV4ConvSmall.mnist(), 128)
    eager.set_batch(*batch)
    eager_losses = []
    for _ in range(3):
        eager.run_eager(after=lambda op: None)  # oxh_program_run_op per group
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
    # the whole program run eagerly (oxh_program_run: the deferred sums too) from the graph's
    # state equals one more group-by-group step
    eager.run_eager(after=lambda op: None)
    graph.run_eager()
    assert graph.loss_value() == eager.loss_value()
    assert graph.steps_taken() == 4
    for i, (a, b) in enumerate(zip(_state(eager), _state(graph))):
        assert_bitexact(b, a, f"state tensor {i} (program run)")
    grads = [op.by_role["gradient"] for s in (eager, graph) for op in s.ops if op.kind == "adamw"]
    assert len(grads) == 2 and len(grads[0]) == 186
    for i, (a, b) in enumerate(zip(*grads)):
        assert_bitexact(host(b), host(a), f"parameter gradient {i}")


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
