"""Host-side description of MobileNetV4-Conv-S by the library (no GPU): the reference's own
shape tests (mobilenet_v4.rs:442-466) and the model census."""

import pytest

import oxide_hip as ox
import training as T


def test_conv_small_matches_supplement_table_11_shapes():
    """mobilenet_v4.rs:442-459."""
    d = T.MobileNetV4ConvSmall.describe(1000, 3, 224, batch=1)
    shapes = d["block_shapes"]
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
    """mobilenet_v4.rs:461-466: [2, 1, 28, 28] -> [2, 10]."""
    d = T.MobileNetV4ConvSmall.describe(10, 1, 28, batch=2)
    assert d["block_shapes"][-1] == (2, 10)
    assert d["block_shapes"][:3] == [(2, 32, 14, 14), (2, 32, 7, 7), (2, 64, 4, 4)]


def test_mnist_model_census():
    """47 convolutions (weight + bias each) and 46 BatchNorms (gamma + beta each) in visit
    order: 186 parameter tensors, 2 517 802 values."""
    d = T.MobileNetV4ConvSmall.describe(10, 1, 28)
    assert d["parameters"] == 2 * 47 + 2 * 46 == 186
    assert d["batch_norms"] == 46
    assert d["values"] == 2517802


def test_invalid_configurations():
    with pytest.raises(ox.OxideError) as e:
        T.MobileNetV4ConvSmall.describe(0, 1, 28)
    assert e.value.status == ox.INVALID_SHAPE and "num_classes" in str(e.value)
    with pytest.raises(ox.OxideError):
        T.MobileNetV4ConvSmall.describe(10, 1, 28, batch=0)
