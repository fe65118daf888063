"""MNIST batches gathered on the GPU, the inference-mode forward, and the OXTR round trip of a
trained step (mnist_training.rs:75-170 end to end, on synthetic IDX data)."""

import numpy as np
import pytest
import torch

import data as D
import oracle
import oxide_hip as ox
import training as T
from helpers import assert_bitexact, assert_close, assert_conv_forward, assert_within, host

pytestmark = pytest.mark.gpu


def _dataset(n, seed=4):
    r = np.random.default_rng(seed)
    return (r.integers(0, 256, (n, 784)).astype(np.uint8),
            r.integers(0, 10, n).astype(np.uint8))


def test_device_gather_equals_host_batches():
    images, labels = _dataset(1000)
    split = D.DeviceSplit(images, labels, shuffle=True)
    np.testing.assert_array_equal(split.order_host, oracle.mnist_order(1000, True))
    out_i = torch.empty((128, 1, 28, 28), device="cuda")
    out_l = torch.empty(128, device="cuda")
    for k in range(split.batches(128)):
        split.gather(k, 128, out_i, out_l)
        torch.cuda.synchronize()
        ref_i, ref_l = D.host_batch(images, labels, split.order_host[k * 128:(k + 1) * 128])
        assert_bitexact(host(out_i), ref_i, f"images of batch {k}")
        assert_bitexact(host(out_l), ref_l, f"labels of batch {k}")
    with pytest.raises(ox.OxideError):
        split.gather(split.batches(128), 128, out_i, out_l)


def test_device_gather_out_of_range_index_gives_nan():
    images, labels = _dataset(10)
    split = D.DeviceSplit(images, labels, shuffle=False)
    split.order[3] = 10  # outside the split: NaN image and label, nothing read out of bounds
    out_i = torch.empty((5, 1, 28, 28), device="cuda")
    out_l = torch.empty(5, device="cuda")
    split.gather(0, 5, out_i, out_l)
    torch.cuda.synchronize()
    oi, ol = host(out_i), host(out_l)
    assert np.isnan(oi[3]).all() and np.isnan(ol[3])
    assert not np.isnan(oi[[0, 1, 2, 4]]).any()
    np.testing.assert_array_equal(ol[[0, 1, 2, 4]], labels[[0, 1, 2, 4]].astype(np.float32))


class EvalChecker:
    def __init__(self):
        self.count = 0

    def before(self, op):
        pass

    def after(self, op):
        torch.cuda.synchronize()
        r = {k: host(v) for k, v in op.reads.items()}
        w = {k: host(v) for k, v in op.writes.items()}
        a = op.attrs
        if op.kind == "conv2d_forward":
            assert_conv_forward(w["y"], r["x"], r["weight"], r["bias"], a["stride"],
                                a["padding"], a["groups"], op.name)
        elif op.kind == "batch_norm2d_eval_forward":
            y, _, inv, rm, rv = oracle.bn_forward(r["x"], r["weight"], r["bias"],
                                                  r["running_mean"], r["running_variance"],
                                                  False, 0.1, a["epsilon"])
            assert_bitexact(w["inverse_std"], inv, f"{op.name} running inverse std")
            assert_bitexact(w["y"], y, f"{op.name} y")  # elementwise with the same statistics
        elif op.kind == "relu_forward":
            assert_bitexact(w["y"], oracle.relu(r["x"]), op.name)
        elif op.kind == "add_forward":
            assert_bitexact(w["y"], oracle.add(r["a"], r["b"]), op.name)
        elif op.kind == "avg_pool2d_forward":
            assert_bitexact(w["y"], oracle.avg_pool2d_forward(r["x"], a["kernel"], a["stride"]),
                            op.name)
        else:
            raise AssertionError(op.kind)
        self.count += 1


def test_train_save_load_evaluate(tmp_path):
    """Two training steps on gathered batches, then: device state -> host (sync_to_model) ->
    OXTR file -> load_mnist; the loaded model's inference forward equals the trained step's
    own (shared device tensors) bit for bit, every eval launch matches the oracle, and the
    predictions are the oracle's argmax."""
    images, labels = _dataset(512, seed=6)
    split = D.DeviceSplit(images, labels, shuffle=True)
    model = T.MobileNetV4ConvSmall.mnist()
    step = T.TrainingStep(model, 128)
    for k in range(2):
        step.stream.synchronize()
        split.gather(k, 128, step.input, step.targets, stream=step.stream)
        step.run_eager()
        assert np.isfinite(step.loss_value())
    step.sync_to_model()
    path = tmp_path / "mobilenetv4-mnist.oxtr"
    model.save(path)
    loaded = T.MobileNetV4ConvSmall.load_mnist(path)
    test_i, _ = D.host_batch(images, labels, np.arange(64, dtype=np.uint64))
    shared = T.EvalForward(model, 64, source=step)
    fresh = T.EvalForward(loaded, 64)
    shared.set_images(test_i)
    fresh.set_images(test_i)
    shared.run()
    checker = EvalChecker()
    fresh.run(checker.before, checker.after)
    torch.cuda.synchronize()
    # 47 convolutions, 46 BatchNorms, 32 ReLUs, 10 residual adds; the global pool of the 1 x 1
    # plane is a view (no launch)
    assert checker.count == 47 + 46 + 32 + 10
    assert_bitexact(host(fresh.logits), host(shared.logits), "logits")
    np.testing.assert_array_equal(fresh.predicted_classes(),
                                  oracle.argmax_rows(host(fresh.logits)))


def _model_tensors(model):
    out = [(p.shape, host(p.value)) for p in model.parameters()]
    for bn in model.batch_norms():
        out += [((bn.channels,), host(bn.device_running_mean)),
                ((bn.channels,), host(bn.device_running_variance))]
    return out


def test_model_save_load_round_trip(tmp_path):
    """save() writes parameters (visit order) then each BatchNorm's running mean / variance
    (mobilenet_v4.rs:217-264), byte for byte as the oracle's writer; load_mnist restores them
    and switches to inference mode."""
    model = T.MobileNetV4ConvSmall.mnist()
    r = np.random.default_rng(3)
    for bn in model.batch_norms():
        bn.device_running_mean.copy_from(r.standard_normal(bn.channels).astype(np.float32))
        bn.device_running_variance.copy_from(r.uniform(0.5, 2, bn.channels).astype(np.float32))
    path = tmp_path / "mobilenetv4-mnist.oxtr"
    model.save(path)
    tensors = _model_tensors(model)
    assert len(tensors) == 186 + 2 * 46
    assert path.read_bytes() == oracle.oxtr_bytes(tensors)
    loaded = T.MobileNetV4ConvSmall.load_mnist(path)
    assert loaded.training is False
    for a, b in zip(_model_tensors(loaded), tensors):
        assert tuple(a[0]) == tuple(b[0])
        np.testing.assert_array_equal(a[1], b[1])
    # the deterministic init reached the device unchanged
    p0 = model.parameters()[0]
    np.testing.assert_array_equal(host(p0.value), oracle.initialized_weights([32, 1, 3, 3], 1))


def test_model_load_errors(tmp_path):
    """load_mnist's error kinds (mobilenet_v4.rs:271-321)."""
    tensors = _model_tensors(T.MobileNetV4ConvSmall.mnist())
    path = tmp_path / "m.oxtr"

    def expect(ts, status, text):
        ox.checkpoint_save(path, ts)
        with pytest.raises(ox.OxideError) as e:
            T.MobileNetV4ConvSmall.load_mnist(path)
        assert e.value.status == status and text in str(e.value), str(e.value)

    expect(tensors[:100], ox.EXECUTION, "checkpoint has too few tensors")
    expect(tensors[:186], ox.EXECUTION, "checkpoint has too few buffers")
    expect(tensors + [((1,), np.zeros(1, np.float32))], ox.EXECUTION, "extra tensors")
    bad = list(tensors)
    bad[0] = ((32, 1, 3, 2), np.zeros(192, np.float32))
    expect(bad, ox.INVALID_SHAPE, "checkpoint tensor 0 has a different shape")
    bad = list(tensors)
    bad[0] = ((32, 1, 3, 3), np.zeros(10, np.float32))
    expect(bad, ox.INVALID_SHAPE, "data length does not match the shape")
    bad = list(tensors)
    bad[186] = ((31,), np.zeros(31, np.float32))
    expect(bad, ox.INVALID_SHAPE, "checkpoint buffer 186 shape mismatch")
    # a trainer needs a model in training mode
    ox.checkpoint_save(path, tensors)
    loaded = T.MobileNetV4ConvSmall.load_mnist(path)
    with pytest.raises(ox.OxideError) as e:
        T.TrainingStep(loaded, 4)
    assert e.value.status == ox.EXECUTION
    loaded.train()
    T.TrainingStep(loaded, 4)
