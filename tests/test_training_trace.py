"""Host-side tracing of MobileNetV4-Conv-S (no GPU): the reference's own shape tests
(mobilenet_v4.rs:442-466) and module validation errors (nn.rs)."""

import pytest

import oxide_hip as ox
import training as T


def test_conv_small_matches_supplement_table_11_shapes():
    """mobilenet_v4.rs:442-459."""
    model = T.MobileNetV4ConvSmall.new(1000)
    out, shapes = model.forward_with_shapes(T.Node("input", (), (1, 3, 224, 224)))
    assert out.shape == (1, 1000)
    assert len(shapes) == 19
    assert shapes[0] == (1, 32, 112, 112)
    assert shapes[1] == (1, 32, 56, 56)
    assert shapes[2] == (1, 64, 28, 28)
    assert shapes[3] == (1, 96, 14, 14)
    assert all(s == (1, 96, 14, 14) for s in shapes[3:9])
    assert all(s == (1, 128, 7, 7) for s in shapes[9:15])
    assert shapes[15] == (1, 960, 7, 7)
    assert shapes[16] == (1, 960, 1, 1)
    assert shapes[17] == (1, 1280, 1, 1)
    assert shapes[18] == (1, 1000)


def test_mnist_variant_accepts_grayscale_images():
    """mobilenet_v4.rs:461-466."""
    model = T.MobileNetV4ConvSmall.mnist()
    assert model.forward(T.Node("input", (), (2, 1, 28, 28))).shape == (2, 10)
    with pytest.raises(ox.OxideError):
        model.forward(T.Node("input", (), (2, 3, 28, 28)))


def test_mnist_graph_census():
    """The traced step: 47 convolutions (one per Conv2d), 46 BatchNorms, a residual add per
    stride-1 block with equal channels, parameters in visit order (weight, bias per conv;
    gamma, beta per BatchNorm)."""
    model = T.MobileNetV4ConvSmall.mnist()
    loss = model.forward(T.Node("input", (), (8, 1, 28, 28))).cross_entropy(
        T.Node("targets", (), (8,)))
    ops = [n.op for n in T._topological(loss)]
    assert ops.count("conv2d") == 47 and ops.count("batch_norm2d") == 46
    residual = sum(getattr(b, "residual", False) for b in model.blocks)
    assert ops.count("add") == residual == 10
    params = model.parameters()
    assert len(params) == 2 * 47 + 2 * 46
    assert params[0].shape == (32, 1, 3, 3) and params[1].shape == (32,)
    assert params[-2].shape == (10, 1280, 1, 1)
    # every parameter is reached by the traced graph exactly once
    ids = [n.attrs["param"] for n in T._topological(loss) if n.op == "param"]
    assert sorted(map(id, ids)) == sorted(map(id, params))


def test_module_validation():
    with pytest.raises(ox.OxideError):
        T.Conv2d(3, 4, 3, 1, 2)  # 3 channels do not split into 2 groups
    with pytest.raises(ox.OxideError):
        T.Conv2d(4, 4, 0, 1, 1)
    with pytest.raises(ox.OxideError):
        T.UniversalInvertedBottleneck(8, 8, 16, 3, None, 2)
    with pytest.raises(ox.OxideError):
        T.MobileNetV4ConvSmall(0)
