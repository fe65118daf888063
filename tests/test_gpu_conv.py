"""conv2d forward / input / weight / bias backward and avg_pool2d on the GPU against the oracle
(evaluation.rs:334-445, autograd.rs:412-527) on every MobileNetV4-Conv-S layer kind.

Input gradient, pooling and all but small pointwise forwards sum their terms in the CPU path's
order: bit-exact.  The forward of a small pointwise convolution (four contiguous parts of the
input channels, added in order) and the weight and bias gradients (batch chunks in a fixed
order): |gpu - cpu| <= 1e-5 * sum|terms|."""

import numpy as np
import pytest
import torch

import oracle
import oxide_hip as ox
from helpers import (assert_bitexact, assert_conv_forward, assert_conv_input_gradient,
                     assert_within, host, to_dev)

pytestmark = pytest.mark.gpu

CASES = [
    (2, 1, 28, 28, 32, 3, 2, 1),
    (128, 1, 28, 28, 32, 3, 2, 1),     # config 5 stem at full batch
    (3, 32, 7, 7, 32, 3, 2, 1),
    (2, 64, 4, 4, 64, 5, 1, 64),
    (2, 192, 4, 4, 192, 5, 2, 192),
    (4, 96, 2, 2, 192, 1, 1, 1),
    (3, 12, 6, 5, 8, 3, 1, 4),
    (5, 20, 1, 1, 30, 1, 1, 1),
    (128, 960, 1, 1, 1280, 1, 1, 1),   # config 5's largest layer (split 16 x 16 forward tiles)
    (128, 384, 2, 2, 96, 1, 1, 1),     # split 16 x 16 forward tiles, plane > 1
    # pointwise (1x1, stride 1) product path: k over several 128-slabs, partial 32-tiles,
    # the weight gradient split over (n, p) chunks, plane 1 and plane > 1
    (3, 300, 3, 3, 40, 1, 1, 1),
    (2, 40, 5, 5, 300, 1, 1, 1),
    (64, 16, 8, 8, 24, 1, 1, 1),
    (1, 7, 1, 1, 3, 1, 1, 1),
    (128, 1280, 1, 1, 10, 1, 1, 1),    # config 5's classifier
    (128, 64, 8, 8, 256, 1, 1, 1),     # grids of >= 512 32 x 32 tiles (the others take 16 x 16)
    (128, 100, 4, 4, 300, 1, 1, 1),    # weight gradient on 32 x 32 tiles, ragged in both axes
    (128, 64, 4, 4, 192, 1, 1, 1),     # 6144 8 x 8 serial tiles (over one round): 16 x 16 ones
    (6, 24, 2, 2, 40, 1, 1, 1),        # weight gradient parts of 6 k: float4 slab loads from
                                       # k = 0, 12 (ragged), scalar ones from k = 6, 18
    (2, 6, 7, 7, 4, 1, 2, 1),          # 1x1 with stride 2: direct path
    # ungrouped 3x3 / 5x5: per-image LDS staging (every K, S pair; ragged channel tiles), and a
    # plane too large to stage (per-thread tap kernels)
    (128, 32, 7, 7, 96, 3, 2, 1),      # config 5's second fused-IB convolution at full batch
    (5, 24, 6, 6, 40, 3, 1, 1),
    (3, 20, 10, 10, 24, 3, 2, 1),      # matrix-core forward: 2 position tiles x 2 channel parts
    (2, 16, 9, 9, 64, 5, 2, 1),        # 5 x 5 stride-2 input gradient staging 64 weights per thread
    (2, 18, 6, 6, 20, 3, 1, 1),        # matrix-core forward: channels not multiples of 4 / 16
    (4, 16, 9, 7, 24, 5, 1, 1),
    (3, 8, 11, 10, 12, 5, 2, 1),
    (2, 64, 20, 20, 16, 3, 1, 1),
]


@pytest.mark.parametrize("case", CASES)
def test_conv2d_matches_oracle(module, dev, case):
    n, cin, h, w, cout, k, s, groups = case
    pad = k // 2
    r = np.random.default_rng(hash(case) & 0xFFFFFFFF)
    x = r.standard_normal((n, cin, h, w)).astype(np.float32)
    wt = (r.standard_normal((cout, cin // groups, k, k)) * 0.3).astype(np.float32)
    b = r.standard_normal(cout).astype(np.float32)
    shape = ox.conv2d_shape(n, cin, h, w, cout, k, s, pad, groups)
    oh, ow = ox.conv2d_output_size(shape)
    g = r.standard_normal((n, cout, oh, ow)).astype(np.float32)
    dx_, dw_, db_, dg_ = to_dev(x, dev), to_dev(wt, dev), to_dev(b, dev), to_dev(g, dev)
    y = torch.empty((n, cout, oh, ow), device=dev)
    gx, gw, gb = torch.empty_like(dx_), torch.empty_like(dw_), torch.empty_like(db_)
    module.conv2d_forward(shape, dx_, dw_, db_, y)
    module.conv2d_input_backward(shape, dg_, dw_, gx)
    module.conv2d_weight_backward(shape, dg_, dx_, gw)
    module.conv2d_bias_backward(shape, dg_, gb)
    torch.cuda.synchronize()
    assert_conv_forward(host(y), x, wt, b, s, pad, groups, "forward")
    rdx, rdw, rdb = oracle.conv2d_backward(g, x, wt, s, pad, groups)
    assert_conv_input_gradient(host(gx), g, wt, s, pad, groups, x.shape, what="input gradient")
    # weight / bias gradient conditioning bounds from the magnitudes of their terms
    abs_dw = oracle.conv2d_backward(np.abs(g), np.abs(x), np.abs(wt), s, pad, groups)[1]
    assert_within(host(gw), rdw, 1e-5 * abs_dw.astype(np.float64) + 1e-7, "weight gradient")
    assert_within(host(gb), rdb, 1e-5 * np.abs(g).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                  "bias gradient")


@pytest.mark.parametrize("case", [(2, 64, 4, 4, 64, 5, 1, 64), (3, 12, 6, 5, 8, 3, 1, 4),
                                  (4, 96, 2, 2, 192, 1, 1, 1), (128, 64, 8, 8, 256, 1, 1, 1),
                                  (2, 6, 7, 7, 4, 1, 2, 1)])
@pytest.mark.parametrize("in_place", [False, True])
def test_conv2d_input_backward_accumulate(module, dev, case, in_place):
    """Input gradient plus an addend in the same pass (a residual input's two gradient
    contributions): bit-equal to the oracle's input gradient followed by the accumulation add,
    on the direct and product paths, with the addend a separate buffer or the output itself."""
    n, cin, h, w, cout, k, s, groups = case
    pad = k // 2
    r = np.random.default_rng(hash(case) & 0xFFFFFF)
    shape = ox.conv2d_shape(n, cin, h, w, cout, k, s, pad, groups)
    oh, ow = ox.conv2d_output_size(shape)
    wt = (r.standard_normal((cout, cin // groups, k, k)) * 0.3).astype(np.float32)
    g = r.standard_normal((n, cout, oh, ow)).astype(np.float32)
    addend = r.standard_normal((n, cin, h, w)).astype(np.float32)
    dw_, dg_, da_ = to_dev(wt, dev), to_dev(g, dev), to_dev(addend, dev)
    out = da_ if in_place else torch.empty_like(da_)
    module.conv2d_input_backward_accumulate(shape, dg_, dw_, da_, out)
    torch.cuda.synchronize()
    assert_conv_input_gradient(host(out), g, wt, s, pad, groups, (n, cin, h, w), addend,
                               "accumulated input gradient")
    with pytest.raises(ox.OxideError):
        module.conv2d_input_backward_accumulate(shape, dg_, dw_, None, out)


@pytest.mark.parametrize("case", [
    (128, 96, 4, 4, 192, 1, 1, 1),     # config-5 shapes: both products in one launch (plane > 1)
    (128, 512, 1, 1, 128, 1, 1, 1),    # plane 1: the other operand layouts, one launch
    (6, 24, 2, 2, 40, 1, 1, 1),        # float4 and scalar slab loads in one paired launch
    (128, 64, 8, 8, 256, 1, 1, 1),     # chunked weight gradient, grids too large to pair
    (128, 960, 1, 1, 1280, 1, 1, 1),
    (128, 1280, 1, 1, 10, 1, 1, 1),    # the classifier: the bias gradient in the paired launch
    (1, 1, 3, 3, 5, 1, 1, 1),          # one input channel: layouts outside the paired set
    (3, 12, 6, 5, 8, 3, 1, 4),         # grouped 3 x 3 and ungrouped 3 x 3: the separate kernels
    (128, 32, 7, 7, 96, 3, 2, 1),
])
@pytest.mark.parametrize("variant", ["plain", "bias", "addend", "addend in place"])
def test_conv2d_backward_equals_separate_calls(module, dev, case, variant):
    """oxh_conv2d_backward (the whole VJP in one call) writes exactly what the separate weight,
    bias and input (or input + addend) backward entry points write."""
    n, cin, h, w, cout, k, s, groups = case
    pad = k // 2
    r = np.random.default_rng(hash((case, variant)) & 0xFFFFFF)
    shape = ox.conv2d_shape(n, cin, h, w, cout, k, s, pad, groups)
    oh, ow = ox.conv2d_output_size(shape)
    x = to_dev(r.standard_normal((n, cin, h, w)).astype(np.float32), dev)
    wt = to_dev((r.standard_normal((cout, cin // groups, k, k)) * 0.3).astype(np.float32), dev)
    g = to_dev(r.standard_normal((n, cout, oh, ow)).astype(np.float32), dev)
    addend = to_dev(r.standard_normal((n, cin, h, w)).astype(np.float32), dev)
    ref_dx, ref_dw, ref_db = torch.empty_like(x), torch.empty_like(wt), torch.empty(cout, device=dev)
    if variant.startswith("addend"):
        module.conv2d_input_backward_accumulate(shape, g, wt, addend, ref_dx)
    else:
        module.conv2d_input_backward(shape, g, wt, ref_dx)
    module.conv2d_weight_backward(shape, g, x, ref_dw)
    module.conv2d_bias_backward(shape, g, ref_db)
    dx = addend.clone() if variant == "addend in place" else torch.full_like(x, float("nan"))
    dw, db = torch.full_like(wt, float("nan")), torch.full((cout,), float("nan"), device=dev)
    module.conv2d_backward(shape, g, x, wt, dx, dw, db if variant == "bias" else None,
                           addend=(dx if variant == "addend in place" else
                                   addend if variant == "addend" else None))
    torch.cuda.synchronize()
    assert_bitexact(host(dx), host(ref_dx), "input gradient")
    assert_bitexact(host(dw), host(ref_dw), "weight gradient")
    if variant == "bias":
        assert_bitexact(host(db), host(ref_db), "bias gradient")
    else:
        assert np.isnan(host(db)).all()  # not written
    with pytest.raises(ox.OxideError):  # the input gradient may not overlap the gradient
        module.conv2d_backward(shape, g, x, wt, g if g.numel() >= x.numel() else x, dw)
    if variant == "bias" and dw.numel() >= cout:
        with pytest.raises(ox.OxideError):  # nor the bias gradient the weight gradient
            module.conv2d_backward(shape, g, x, wt, dx, dw, dw.view(-1)[:cout])


@pytest.mark.parametrize("case", [
    (128, 1, 28, 28, 32, 3, 2, 1),     # config 5's stem: bias in the weight launch, chunked
    (128, 32, 7, 7, 96, 3, 2, 1),      # one pair per thread (no position ranges)
    (2, 18, 6, 6, 20, 3, 1, 1),        # ragged channel tile, one chunk per image
    (1, 5, 8, 8, 6, 5, 2, 1),          # one chunk: the sums written in place
    (3, 12, 6, 5, 8, 3, 1, 4),         # grouped: the separate bias kernel
    (4, 96, 2, 2, 192, 1, 1, 1),       # pointwise: the separate kernels
])
def test_conv2d_parameter_backward(module, dev, case):
    """oxh_conv2d_backward without an input gradient: the weight gradient bit-equal to
    oxh_conv2d_weight_backward's, the bias gradient (summed in the weight gradient's launches
    where the per-image kernels take the shape) within 1e-5 * sum|terms| of the oracle."""
    n, cin, h, w, cout, k, s, groups = case
    pad = k // 2
    r = np.random.default_rng(hash(case) & 0xFFFFFF)
    shape = ox.conv2d_shape(n, cin, h, w, cout, k, s, pad, groups)
    oh, ow = ox.conv2d_output_size(shape)
    x = r.standard_normal((n, cin, h, w)).astype(np.float32)
    wt = (r.standard_normal((cout, cin // groups, k, k)) * 0.3).astype(np.float32)
    g = r.standard_normal((n, cout, oh, ow)).astype(np.float32)
    dx_, dw_, dg_ = to_dev(x, dev), to_dev(wt, dev), to_dev(g, dev)
    ref_dw = torch.empty_like(dw_)
    module.conv2d_weight_backward(shape, dg_, dx_, ref_dw)
    dw, db = torch.full_like(dw_, float("nan")), torch.full((cout,), float("nan"), device=dev)
    module.conv2d_backward(shape, dg_, dx_, dw_, None, dw, db)
    torch.cuda.synchronize()
    assert_bitexact(host(dw), host(ref_dw), "weight gradient")
    assert_within(host(db), oracle.conv2d_bias_backward(g),
                  1e-5 * np.abs(g).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7,
                  "bias gradient")
    with pytest.raises(ox.OxideError):  # an addend needs an input gradient
        module.conv2d_backward(shape, dg_, dx_, dw_, None, dw, db, addend=dx_)


@pytest.mark.parametrize("shape,kernel,stride", [((2, 3, 4, 4), (2, 2), (2, 2)),
                                                 ((128, 960, 1, 1), (1, 1), (1, 1)),
                                                 ((2, 5, 7, 7), (7, 7), (7, 7)),
                                                 ((1, 2, 5, 6), (3, 2), (1, 2))])
def test_avg_pool2d_matches_oracle(module, dev, shape, kernel, stride):
    r = np.random.default_rng(3)
    x = r.standard_normal(shape).astype(np.float32)
    ps = ox.Pool2dShape(*shape, kernel[0], kernel[1], stride[0], stride[1])
    ref = oracle.avg_pool2d_forward(x, kernel, stride)
    y = torch.empty(ref.shape, device=dev)
    module.avg_pool2d_forward(ps, to_dev(x, dev), y)
    g = r.standard_normal(ref.shape).astype(np.float32)
    dx = torch.empty(shape, device=dev)
    module.avg_pool2d_backward(ps, to_dev(g, dev), dx)
    torch.cuda.synchronize()
    assert_bitexact(host(y), ref, "pool forward")
    assert_bitexact(host(dx), oracle.avg_pool2d_backward(g, shape, kernel, stride),
                    "pool backward")


def test_conv_reference_kat(module, dev):
    """tensor/mod.rs:586-614 on the GPU."""
    x = np.arange(1, 10, dtype=np.float32).reshape(1, 1, 3, 3)
    shape = ox.conv2d_shape(1, 1, 3, 3, 1, 2, 1, 0, 1)
    y = torch.empty((1, 1, 2, 2), device=dev)
    module.conv2d_forward(shape, to_dev(x, dev), torch.ones((1, 1, 2, 2), device=dev),
                          torch.zeros(1, device=dev), y)
    dwx = np.arange(1, 9, dtype=np.float32).reshape(1, 2, 2, 2)
    dshape = ox.conv2d_shape(1, 2, 2, 2, 2, 1, 1, 0, 2)
    dy = torch.empty((1, 2, 2, 2), device=dev)
    module.conv2d_forward(dshape, to_dev(dwx, dev), to_dev(np.array([2.0, 3.0], np.float32)
                                                          .reshape(2, 1, 1, 1), dev),
                          torch.zeros(2, device=dev), dy)
    torch.cuda.synchronize()
    assert host(y).ravel().tolist() == [12.0, 16.0, 24.0, 28.0]
    assert host(dy).ravel().tolist() == [2, 4, 6, 8, 15, 18, 21, 24]


def test_adamw_step_counter_matches_host_corrections(module, dev, rng):
    """oxh_adamw_multi_tensor_step: the device step counter gives the same bit-exact update as
    host-computed corrections, on consecutive steps."""
    n = 3000
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    dp, dg = to_dev(p, dev), to_dev(g, dev)
    dm, dv = torch.zeros_like(dp), torch.zeros_like(dp)
    step = torch.zeros(1, dtype=torch.int32, device=dev)
    pr, mr, vr = p, np.zeros_like(p), np.zeros_like(p)
    for t in range(1, 4):
        module.adamw_multi_tensor_step(1e-3, 1e-4, 0.9, 0.999, 1e-8, step, [(dp, dg, dm, dv)])
        pr, mr, vr = oracle.adamw_update(pr, g, mr, vr, t, 1e-3, 1e-4)
        torch.cuda.synchronize()
        assert int(host(step)[0]) == t
        assert_bitexact(host(dp), pr, f"param step {t}")
        assert_bitexact(host(dv), vr, f"v step {t}")
