"""Depthwise ConvNormAct (nn.rs:362-395 with groups == channels) in one launch per direction
(oxh_depthwise_conv_batch_norm_{forward,backward}_train) against the separate entry points it
replaces and against the oracle.

Bars: the fused outputs equal the separate launches' bit for bit (convolution output, BatchNorm
output and statistics, running statistics, BatchNorm gradients, the convolution's output,
bias and input gradients; the weight gradient too where the separate depthwise weight kernel
also runs 256 threads, i.e. more than 128 channels).  Against the oracle: convolution output
and input gradient bit-exact, BatchNorm within the north star's 1e-5 relative (conditioning
bound for cancelling sums), weight / bias gradients within 1e-5 * sum|terms|."""

import numpy as np
import pytest
import torch

import oracle
import oxide_hip as ox
from helpers import (assert_bitexact, assert_within, check_batch_norm_backward,
                     check_batch_norm_forward, host, to_dev)

pytestmark = pytest.mark.gpu

# (batch, channels, height, width, kernel, stride, padding): the MNIST MobileNetV4's depthwise
# layers (nn.rs:459-485; 4x4 after the stem and two fused blocks), then ragged, minimal and
# maximal shapes
SHAPES = [
    (128, 64, 4, 4, 5, 1, 2),    # first UIB start depthwise
    (128, 192, 4, 4, 5, 2, 2),   # first UIB middle depthwise, stride 2
    (128, 192, 2, 2, 3, 1, 1),
    (128, 96, 2, 2, 3, 1, 1),
    (128, 576, 2, 2, 3, 2, 1),   # stride 2 to 1x1
    (128, 512, 1, 1, 5, 1, 2),   # 1x1 planes: one valid tap (the centre-only kernels)
    (128, 64, 1, 1, 3, 2, 1),
    (3, 5, 7, 6, 3, 2, 1),       # ragged, output 4 x 3
    (2, 3, 9, 9, 5, 1, 2),
    (16, 4, 4, 4, 3, 1, 0),      # no padding
    (8, 6, 4, 4, 3, 2, 1),       # 4x4 planes, 3x3 stride 2 (one thread per image)
    (2, 1, 1, 1, 3, 1, 1),       # two values per channel (the minimum)
    (128, 3, 4, 4, 5, 1, 2),     # 2048 output values per channel (the maximum)
    (32, 130, 16, 16, 3, 2, 1),  # 8192 input values per channel (the maximum), 8x8 output
]


def _shape(b, c, h, w, k, s, p):
    return ox.conv2d_shape(b, c, h, w, c, k, s, p, c)


def _case(r, b, c, h, w, k, s, p):
    sh = _shape(b, c, h, w, k, s, p)
    oh, ow = ox.conv2d_output_size(sh)
    d = dict(
        x=r.standard_normal((b, c, h, w)).astype(np.float32),
        cw=r.uniform(-0.5, 0.5, (c, 1, k, k)).astype(np.float32),
        cb=r.uniform(-0.2, 0.2, c).astype(np.float32),
        gamma=r.uniform(0.5, 1.5, c).astype(np.float32),
        beta=r.uniform(-0.1, 0.1, c).astype(np.float32),
        rm=r.uniform(-0.5, 0.5, c).astype(np.float32),
        rv=r.uniform(0.5, 2.0, c).astype(np.float32),
        g=r.standard_normal((b, c, oh, ow)).astype(np.float32),
        addend=r.standard_normal((b, c, h, w)).astype(np.float32))
    return sh, (b, c, oh, ow), d


def _fused(module, dev, sh, oshape, d, relu, with_addend):
    t = {k: to_dev(v, dev) for k, v in d.items()}
    c = oshape[1]
    o = dict(conv=torch.empty(oshape, device=dev), y=torch.empty(oshape, device=dev),
             mean=torch.empty(c, device=dev), inv=torch.empty(c, device=dev))
    module.depthwise_conv_batch_norm_forward_train(
        sh, relu, 0.1, 1e-5, t["x"], t["cw"], t["cb"], o["conv"], t["gamma"], t["beta"],
        t["rm"], t["rv"], o["mean"], o["inv"], o["y"])
    o.update(gconv=torch.empty(oshape, device=dev), dgamma=torch.empty(c, device=dev),
             dbeta=torch.empty(c, device=dev), dcb=torch.empty(c, device=dev),
             dcw=torch.empty_like(t["cw"]), dx=torch.empty_like(t["x"]))
    module.depthwise_conv_batch_norm_backward_train(
        sh, t["g"], o["y"] if relu else None, o["conv"], t["gamma"], o["mean"], o["inv"],
        t["x"], t["cw"], t["addend"] if with_addend else None, o["gconv"], o["dgamma"],
        o["dbeta"], o["dcb"], o["dcw"], o["dx"])
    torch.cuda.synchronize()
    o.update(rm=t["rm"], rv=t["rv"])
    return {k: host(v) for k, v in o.items()}


def _separate(module, dev, sh, oshape, d, relu, with_addend):
    t = {k: to_dev(v, dev) for k, v in d.items()}
    c = oshape[1]
    o = dict(conv=torch.empty(oshape, device=dev), y=torch.empty(oshape, device=dev),
             mean=torch.empty(c, device=dev), inv=torch.empty(c, device=dev))
    module.conv2d_forward(sh, t["x"], t["cw"], t["cb"], o["conv"])
    bn = module.batch_norm_relu_forward_train if relu else module.batch_norm_forward_train
    bn(o["conv"], t["gamma"], t["beta"], t["rm"], t["rv"], o["mean"], o["inv"], o["y"])
    o.update(gconv=torch.empty(oshape, device=dev), dgamma=torch.empty(c, device=dev),
             dbeta=torch.empty(c, device=dev), dcb=torch.empty(c, device=dev),
             dcw=torch.empty_like(t["cw"]), dx=torch.empty_like(t["x"]))
    module.conv_batch_norm_backward_train(t["g"], o["y"] if relu else None, o["conv"],
                                          t["gamma"], o["mean"], o["inv"], o["gconv"],
                                          o["dgamma"], o["dbeta"], o["dcb"])
    module.conv2d_weight_backward(sh, o["gconv"], t["x"], o["dcw"])
    if with_addend:
        module.conv2d_input_backward_accumulate(sh, o["gconv"], t["cw"], t["addend"], o["dx"])
    else:
        module.conv2d_input_backward(sh, o["gconv"], t["cw"], o["dx"])
    torch.cuda.synchronize()
    o.update(rm=t["rm"], rv=t["rv"])
    return {k: host(v) for k, v in o.items()}


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("relu", [True, False])
def test_fused_matches_oracle(module, dev, shape, relu):
    b, c, h, w, k, s, p = shape
    r = np.random.default_rng(hash((shape, relu)) & 0xFFFFFF)
    sh, oshape, d = _case(r, *shape)
    assert ox.depthwise_conv_batch_norm_supported(sh)
    with_addend = bool(relu)
    out = _fused(module, dev, sh, oshape, d, relu, with_addend)
    assert_bitexact(out["conv"], oracle.conv2d_forward(d["x"], d["cw"], d["cb"], s, p, c),
                    "conv output")
    check_batch_norm_forward(dict(y=out["y"], mean=out["mean"], inv=out["inv"], rm=out["rm"],
                                  rv=out["rv"]), out["conv"], d["gamma"], d["beta"], d["rm"],
                             d["rv"], relu=relu)
    g = oracle.relu_backward(d["g"], out["y"]) if relu else d["g"]
    check_batch_norm_backward(dict(dx=out["gconv"], dw=out["dgamma"], db=out["dbeta"]), g,
                              out["conv"], d["gamma"], out["mean"], out["inv"])
    gc = out["gconv"]
    rdx, rdw, rdb = oracle.conv2d_backward(gc, d["x"], d["cw"], s, p, c)
    if with_addend:
        rdx = oracle.accumulate(d["addend"], rdx)
    assert_bitexact(out["dx"], rdx, "input gradient")
    abs_dw = oracle.conv2d_backward(np.abs(gc), np.abs(d["x"]), np.abs(d["cw"]), s, p, c)[1]
    assert_within(out["dcw"], rdw, 1e-5 * abs_dw.astype(np.float64) + 1e-7, "weight gradient")
    assert_within(out["dcb"], rdb, 1e-5 * np.abs(gc).astype(np.float64).sum(axis=(0, 2, 3))
                  + 1e-7, "bias gradient")


def _output_plane(shape):
    b, c, h, w, k, s, p = shape
    return ((h + 2 * p - k) // s + 1) * ((w + 2 * p - k) // s + 1)


@pytest.mark.parametrize("shape", [sh for sh in SHAPES
                                   if sh[2] * sh[3] < 256 and _output_plane(sh) < 64])
@pytest.mark.parametrize("relu", [True, False])
def test_fused_matches_separate_launches_bitwise(module, dev, shape, relu):
    """Planes whose separate BatchNorm runs the one-block-per-channel kernel (output planes
    under 64 values; larger ones take the reduce + map path, whose sums are ordered
    differently): every output bit-equal to the separate launches'."""
    b, c, h, w, k, s, p = shape
    r = np.random.default_rng(hash((shape, relu, 1)) & 0xFFFFFF)
    sh, oshape, d = _case(r, *shape)
    assert oshape[2] * oshape[3] == _output_plane(shape)
    fused = _fused(module, dev, sh, oshape, d, relu, True)
    sep = _separate(module, dev, sh, oshape, d, relu, True)
    names = ["conv", "y", "mean", "inv", "rm", "rv", "gconv", "dgamma", "dbeta", "dcb", "dx"]
    if c > 128:  # the separate depthwise weight kernel runs 256 threads (1024 for <= 128)
        names.append("dcw")
    for n in names:
        np.testing.assert_array_equal(fused[n], sep[n], err_msg=n)


def test_optional_outputs_and_in_place_addend(module, dev):
    """No conv output gradient and no input gradient: the other outputs are unchanged; the
    addend may be the input gradient itself (accumulate in place)."""
    shape = (128, 192, 2, 2, 3, 1, 1)
    r = np.random.default_rng(11)
    sh, oshape, d = _case(r, *shape)
    ref = _fused(module, dev, sh, oshape, d, True, True)
    t = {k: to_dev(v, dev) for k, v in d.items()}
    y, conv = to_dev(ref["y"], dev), to_dev(ref["conv"], dev)
    mean, inv = to_dev(ref["mean"], dev), to_dev(ref["inv"], dev)
    c = shape[1]
    outs = [torch.empty(c, device=dev) for _ in range(3)]
    dcw = torch.empty_like(t["cw"])
    module.depthwise_conv_batch_norm_backward_train(sh, t["g"], y, conv, t["gamma"], mean, inv,
                                                    t["x"], t["cw"], None, None, *outs, dcw,
                                                    None)
    inplace = t["addend"].clone()
    module.depthwise_conv_batch_norm_backward_train(sh, t["g"], y, conv, t["gamma"], mean, inv,
                                                    t["x"], t["cw"], inplace, None, *outs, dcw,
                                                    inplace)
    torch.cuda.synchronize()
    for got, n in zip(outs, ["dgamma", "dbeta", "dcb"]):
        np.testing.assert_array_equal(host(got), ref[n], err_msg=n)
    np.testing.assert_array_equal(host(dcw), ref["dcw"])
    np.testing.assert_array_equal(host(inplace), ref["dx"])


def test_unsupported_shapes_are_rejected(module, dev):
    ok = _shape(128, 64, 4, 4, 5, 1, 2)
    assert ox.depthwise_conv_batch_norm_supported(ok)
    bad = [ox.conv2d_shape(128, 64, 4, 4, 64, 5, 1, 2, 32),   # grouped, not depthwise
           ox.conv2d_shape(128, 64, 4, 4, 128, 5, 1, 2, 64),  # channel multiplier 2
           _shape(128, 64, 8, 8, 3, 1, 1),                     # 8192 output values
           _shape(64, 4, 16, 16, 3, 2, 1),                     # 16384 input values
           _shape(2, 4, 9, 9, 7, 1, 3),                        # 7x7 kernel
           _shape(2, 4, 9, 9, 3, 3, 1),                        # stride 3
           _shape(1, 4, 1, 1, 3, 1, 1)]                        # one value per channel
    for sh in bad:
        assert not ox.depthwise_conv_batch_norm_supported(sh)
    sh = bad[2]
    x = torch.zeros(128, 64, 8, 8, device=dev)
    v = torch.zeros(64, device=dev)
    with pytest.raises(ox.OxideError) as e:
        module.depthwise_conv_batch_norm_forward_train(sh, True, 0.1, 1e-5, x, x, v, x, v, v, v,
                                                       v, v, v, x)
    assert e.value.status == ox.INVALID_SHAPE


# (batch, channels, height, width, kernel, stride, padding) of depthwise layers fed by a
# BatchNorm (+ ReLU): the MNIST MobileNetV4's first UIB start and expand BatchNorms before their
# depthwise layers, 4x4 planes under 3x3 kernels (the backward of a 4x4 plane forms its input
# gradient with one thread per image), then ragged and minimal shapes (at most 2048 input
# values per channel)
PRE_SHAPES = [
    (128, 64, 4, 4, 5, 1, 2),
    (128, 192, 4, 4, 5, 2, 2),
    (8, 6, 4, 4, 3, 1, 1),
    (8, 6, 4, 4, 3, 2, 1),
    (128, 192, 2, 2, 3, 1, 1),
    (128, 576, 2, 2, 3, 2, 1),
    (128, 512, 1, 1, 5, 1, 2),
    (3, 5, 7, 6, 3, 2, 1),
    (2, 1, 1, 1, 3, 1, 1),
]


@pytest.mark.parametrize("case", PRE_SHAPES)
@pytest.mark.parametrize("pre_relu,relu,residual", [(True, True, False), (False, True, False),
                                                    (True, False, False), (False, True, True),
                                                    (False, False, True)])
def test_batch_norm_feeding_depthwise_layer_equals_separate_launches(module, dev, case, pre_relu,
                                                                     relu, residual):
    """oxh_batch_norm_depthwise_conv_batch_norm_{forward,backward}_train: the BatchNorm (+ ReLU,
    or + a residual add) in front of a depthwise ConvNormAct run inside that layer's launches
    writes exactly what the separate BatchNorm and depthwise-layer launches write (the same
    channel arithmetic), in both directions, with the layer input's other gradient
    contributions (an addend) folded in where there is a residual; the BatchNorm in front
    against the oracle too."""
    r = np.random.default_rng(hash((case, pre_relu, relu, residual)) & 0xFFFFFF)
    sh, oshape, d = _case(r, *case)
    b, c = case[0], case[1]
    ishape = (b, c, case[2], case[3])
    y1 = (r.standard_normal(ishape) * 1.5 + 0.3).astype(np.float32)
    g1 = r.uniform(0.5, 1.5, c).astype(np.float32)
    b1 = r.uniform(-0.3, 0.3, c).astype(np.float32)
    rm1 = r.uniform(-0.5, 0.5, c).astype(np.float32)
    rv1 = r.uniform(0.5, 2.0, c).astype(np.float32)
    res = r.standard_normal(ishape).astype(np.float32)
    other = r.standard_normal(ishape).astype(np.float32)  # the input's other contributions
    t = {k: to_dev(v, dev) for k, v in d.items()}
    e = lambda s: torch.empty(s, device=dev)  # noqa: E731

    def run(fused):
        s = dict(y1=to_dev(y1, dev), rm1=to_dev(rm1, dev), rv1=to_dev(rv1, dev),
                 rm2=t["rm"].clone(), rv2=t["rv"].clone(), sm1=e(c), si1=e(c), a1=e(ishape),
                 conv=e(oshape), y2=e(oshape), sm2=e(c), si2=e(c), gconv=e(oshape),
                 dg2=e(c), db2=e(c), dcb=e(c), dcw=torch.empty_like(t["cw"]), dg1=e(c),
                 db1=e(c), dy1=e(ishape), dsum=e(c), da1=e(ishape))
        g1d, b1d = to_dev(g1, dev), to_dev(b1, dev)
        resd, otherd = (to_dev(res, dev), to_dev(other, dev)) if residual else (None, None)
        if fused:
            module.batch_norm_depthwise_conv_batch_norm_forward_train(
                sh, dict(relu=pre_relu, momentum=0.1, epsilon=1e-5, x=s["y1"], weight=g1d,
                         bias=b1d, residual=resd, running_mean=s["rm1"],
                         running_variance=s["rv1"], saved_mean=s["sm1"],
                         saved_inverse_std=s["si1"], out=s["a1"]),
                dict(relu=relu, momentum=0.1, epsilon=1e-5, conv_weight=t["cw"],
                     conv_bias=t["cb"], conv_out=s["conv"], weight=t["gamma"], bias=t["beta"],
                     running_mean=s["rm2"], running_variance=s["rv2"], saved_mean=s["sm2"],
                     saved_inverse_std=s["si2"], out=s["y2"]))
            module.batch_norm_depthwise_conv_batch_norm_backward_train(
                sh, dict(gradient=t["g"], relu_out=s["y2"] if relu else None, conv_out=s["conv"],
                         weight=t["gamma"], saved_mean=s["sm2"], saved_inverse_std=s["si2"],
                         conv_in=s["a1"], conv_weight=t["cw"], conv_out_gradient=s["gconv"],
                         weight_gradient=s["dg2"], bias_gradient=s["db2"],
                         conv_bias_gradient=s["dcb"], conv_weight_gradient=s["dcw"],
                         addend=otherd, conv_in_gradient=s["da1"] if residual else None),
                dict(relu=pre_relu, x=s["y1"], weight=g1d, saved_mean=s["sm1"],
                     saved_inverse_std=s["si1"], weight_gradient=s["dg1"], bias_gradient=s["db1"],
                     input_gradient=s["dy1"], input_gradient_sum=s["dsum"]))
        else:
            if residual:
                module.batch_norm_add_forward_train(s["y1"], g1d, b1d, s["rm1"], s["rv1"],
                                                    s["sm1"], s["si1"], resd, s["a1"])
            else:
                fwd = (module.batch_norm_relu_forward_train if pre_relu
                       else module.batch_norm_forward_train)
                fwd(s["y1"], g1d, b1d, s["rm1"], s["rv1"], s["sm1"], s["si1"], s["a1"])
            module.depthwise_conv_batch_norm_forward_train(
                sh, relu, 0.1, 1e-5, s["a1"], t["cw"], t["cb"], s["conv"], t["gamma"], t["beta"],
                s["rm2"], s["rv2"], s["sm2"], s["si2"], s["y2"])
            module.depthwise_conv_batch_norm_backward_train(
                sh, t["g"], s["y2"] if relu else None, s["conv"], t["gamma"], s["sm2"], s["si2"],
                s["a1"], t["cw"], otherd, s["gconv"], s["dg2"], s["db2"], s["dcb"], s["dcw"],
                s["da1"])
            module.conv_batch_norm_backward_train(
                s["da1"], s["a1"] if pre_relu else None, s["y1"], g1d, s["sm1"], s["si1"],
                s["dy1"], s["dg1"], s["db1"], s["dsum"])
        torch.cuda.synchronize()
        return {k: host(v) for k, v in s.items()}

    fused, separate = run(True), run(False)
    for k in separate:
        if k == "da1" and not residual:
            continue  # not formed by the fused launch without a residual
        assert_bitexact(fused[k], separate[k], k)
    # the BatchNorm in front against the oracle (its statistics and output)
    bn_out = fused["a1"] - res if residual else fused["a1"]
    if not residual:
        check_batch_norm_forward(dict(y=bn_out, mean=fused["sm1"], inv=fused["si1"],
                                      rm=fused["rm1"], rv=fused["rv1"]),
                                 y1, g1, b1, rm1, rv1, relu=pre_relu)
