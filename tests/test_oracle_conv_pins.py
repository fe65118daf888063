"""Pins the oracle's conv2d / avg_pool2d restatement (evaluation.rs:334-445,
autograd.rs:412-527): the reference's own known-answer test, and torch float64 conv2d /
avg_pool2d with autograd on grouped, strided and padded shapes like MobileNetV4-Conv-S's
layers, so a swapped index, a wrong padding sign or a dropped term fails."""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle

KAT = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())[
    "grouped_convolution_and_average_pool_evaluate"]
torch = pytest.importorskip("torch")


def f32(x, shape=None):
    a = np.asarray(x, dtype=np.float32)
    return a.reshape(shape) if shape is not None else a


def test_kat_grouped_convolution_and_average_pool():
    out = oracle.conv2d_forward(f32(KAT["conv_input"], KAT["conv_input_shape"]),
                                f32(KAT["conv_weight"], KAT["conv_weight_shape"]),
                                np.zeros(1, np.float32), KAT["conv_stride"], KAT["conv_padding"],
                                KAT["conv_groups"])
    assert list(out.shape) == KAT["conv_expected_shape"]
    assert out.ravel().tolist() == KAT["conv_expected"]
    pooled = oracle.avg_pool2d_forward(f32(KAT["pool_input"], KAT["pool_input_shape"]),
                                       KAT["pool_kernel"], KAT["pool_stride"])
    assert pooled.ravel().tolist() == KAT["pool_expected"]
    dw = oracle.conv2d_forward(f32(KAT["depthwise_input"], KAT["depthwise_input_shape"]),
                               f32(KAT["depthwise_weight"], KAT["depthwise_weight_shape"]),
                               np.zeros(2, np.float32), 1, 0, KAT["depthwise_groups"])
    assert dw.ravel().tolist() == KAT["depthwise_expected"]


# (batch, in, h, w, out, kernel, stride, groups): MNv4-Conv-S MNIST layer kinds
CASES = [
    (2, 1, 28, 28, 32, 3, 2, 1),     # stem 3x3 s2
    (3, 32, 7, 7, 32, 3, 2, 1),      # FusedIB expand, odd input with stride 2
    (2, 64, 4, 4, 64, 5, 1, 64),     # start depthwise 5x5
    (2, 192, 4, 4, 192, 5, 2, 192),  # strided middle depthwise
    (4, 96, 2, 2, 192, 1, 1, 1),     # pointwise expand
    (3, 12, 6, 5, 8, 3, 1, 4),       # generic grouped conv, non-square input
    (5, 20, 1, 1, 30, 1, 1, 1),      # 1x1 spatial (tail of the network)
]


@pytest.mark.parametrize("case", CASES)
def test_conv2d_matches_torch_float64(case):
    n, cin, h, w, cout, k, s, groups = case
    pad = k // 2
    r = np.random.default_rng(hash(case) & 0xFFFFFFFF)
    x = r.standard_normal((n, cin, h, w)).astype(np.float32)
    wt = (r.standard_normal((cout, cin // groups, k, k)) * 0.3).astype(np.float32)
    b = r.standard_normal(cout).astype(np.float32)
    y = oracle.conv2d_forward(x, wt, b, s, pad, groups)
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    tw = torch.tensor(wt, dtype=torch.float64, requires_grad=True)
    tb = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    ty = torch.nn.functional.conv2d(tx, tw, tb, stride=s, padding=pad, groups=groups)
    assert y.shape == tuple(ty.shape)
    # conditioning bound: 1e-5 of the sum of |terms| (fp32 accumulation of up to ~600 terms)
    tabs = torch.nn.functional.conv2d(tx.abs(), tw.abs(), tb.abs(), stride=s, padding=pad,
                                      groups=groups).detach().numpy()
    assert np.all(np.abs(y - ty.detach().numpy()) <= 1e-6 * tabs + 1e-7)
    g = r.standard_normal(y.shape).astype(np.float32)
    ty.backward(torch.tensor(g, dtype=torch.float64))
    dx, dw, db = oracle.conv2d_backward(g, x, wt, s, pad, groups)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(db, tb.grad.numpy(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("shape,kernel,stride", [((2, 3, 4, 4), (2, 2), (2, 2)),
                                                 ((2, 5, 7, 7), (7, 7), (7, 7)),
                                                 ((1, 2, 5, 6), (3, 2), (1, 2)),
                                                 ((3, 4, 1, 1), (1, 1), (1, 1))])
def test_avg_pool2d_matches_torch_float64(shape, kernel, stride):
    r = np.random.default_rng(1)
    x = r.standard_normal(shape).astype(np.float32)
    y = oracle.avg_pool2d_forward(x, kernel, stride)
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    ty = torch.nn.functional.avg_pool2d(tx, kernel, stride)
    np.testing.assert_allclose(y, ty.detach().numpy(), rtol=1e-6, atol=1e-7)
    g = r.standard_normal(y.shape).astype(np.float32)
    ty.backward(torch.tensor(g, dtype=torch.float64))
    dx = oracle.avg_pool2d_backward(g, shape, kernel, stride)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-6, atol=1e-7)


def test_library_init_matches_oracle_restatement():
    """The library's host-side nn.rs:657-674 init equals the oracle's restatement bit for bit
    on every MNv4-Conv-S weight shape kind."""
    import oxide_hip

    for shape, ipg in [([32, 1, 3, 3], 1), ([96, 32, 3, 3], 32), ([192, 1, 5, 5], 1),
                       ([1280, 960, 1, 1], 960), ([10, 1280, 1, 1], 1280)]:
        a = oxide_hip.initialized_weights(shape, ipg)
        b = oracle.initialized_weights(shape, ipg)
        assert np.array_equal(a, b), shape


def test_init_statistical_and_structural_properties():
    """nn.rs:657-674 pinned by what its construction fixes (no reference output holds concrete
    weights): every value is (k / 2^24 * 2 - 1) * sqrt(2 / fan_in) for an integer k in
    [0, 2^24) (24-bit uniforms), the values are uniform on [-scale, scale) (mean 0, variance
    scale^2 / 3, extremes near +-scale), consecutive values are uncorrelated (xorshift64
    13/7/17 stream), and the seed is an XOR fold over the dimensions, so shapes that permute
    the same dimensions draw the same unit stream.  A wrong fan-in, shift, scale or a skipped
    xorshift step fails one of these."""
    shape, ipg = [64, 48, 3, 3], 48
    w32 = oracle.initialized_weights(shape, ipg).ravel()
    scale = np.sqrt(np.float32(2.0) / np.float32(ipg * 9)).astype(np.float32)
    # each value is the fp32 product of some grid point (k / 2^23 - 1) and the scale
    k0 = np.round((w32.astype(np.float64) / float(scale) + 1.0) * 2.0 ** 23)
    on_grid = np.zeros(w32.size, bool)
    for d in (-1, 0, 1):
        k = k0 + d
        v = ((k / 2.0 ** 23) - 1.0).astype(np.float32)  # exact in fp32
        on_grid |= (v * scale == w32) & (k >= 0) & (k < 2 ** 24)
    assert on_grid.all()
    u = w32.astype(np.float64) / float(scale)
    n = u.size
    assert abs(u.mean()) < 4 * np.sqrt(1 / 3 / n)
    assert abs(u.var() - 1 / 3) < 0.02
    assert u.max() > 0.999 and u.min() < -0.999 and np.abs(u).max() <= 1.0
    assert abs(np.corrcoef(u[:-1], u[1:])[0, 1]) < 4 / np.sqrt(n)
    a = oracle.initialized_weights([6, 4, 1, 1], 4).ravel() / np.sqrt(np.float32(2 / 4))
    b = oracle.initialized_weights([4, 6, 1, 1], 6).ravel() / np.sqrt(np.float32(2 / 6))
    np.testing.assert_allclose(a, b, rtol=1e-6)
    c = oracle.initialized_weights([5, 4, 1, 1], 4).ravel()[:20] / np.sqrt(np.float32(2 / 4))
    assert not np.allclose(a[:20], c)
