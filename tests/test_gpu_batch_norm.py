"""BatchNorm2d training forward (statistics, running update, apply) and input / weight / bias
backward on the GPU against the oracle (evaluation.rs:448-597, autograd.rs:315-383), from
tiny shapes with vector and scalar paths up to config 2's [64, 128, 56, 56].

Tolerances (north star: max rel err 1e-5, abs 1e-6 near zero):
  * per-element outputs (y, mean, inverse std, running stats, dx) must meet
    |gpu - cpu| <= max(1e-5 |cpu|, 1e-6), or, where the value is a cancelling sum, the
    conditioning bound |gpu - cpu| <= 1e-5 * (sum of the magnitudes of its terms);
  * channel sums (dweight, dbias) of up to 200 704 terms: the oracle's sequential fp32 sum
    carries rounding error ~1e-3 absolute, so they are checked against the conditioning bound
    1e-5 * sum|terms| versus the oracle, and 1e-6 * sum|terms| versus an fp64 sum of the same
    fp32 terms (the GPU accumulates in fp64).
"""

import json

import numpy as np
import pytest
import torch

import oracle
import oxide_hip as ox
from helpers import (assert_close, assert_within, check_batch_norm_backward,
                     check_batch_norm_forward, host, strict_ok, to_dev)

pytestmark = pytest.mark.gpu


def _case(r, shape, scale=1.0, offset=0.0):
    n, c, h, w = shape
    x = (r.standard_normal(shape) * scale + offset).astype(np.float32)
    gamma = r.uniform(0.5, 1.5, c).astype(np.float32)
    beta = r.uniform(-0.1, 0.1, c).astype(np.float32)
    g = r.standard_normal(shape).astype(np.float32)
    return x, gamma, beta, g


def _run(module, dev, x, gamma, beta, g, rm, rv, momentum=0.1, eps=1e-5):
    c = x.shape[1]
    dx_, dw_, db_, dg_ = to_dev(x, dev), to_dev(gamma, dev), to_dev(beta, dev), to_dev(g, dev)
    drm, drv = to_dev(rm, dev), to_dev(rv, dev)
    y = torch.empty_like(dx_)
    mean, inv = torch.empty(c, device=dev), torch.empty(c, device=dev)
    module.batch_norm_forward_train(dx_, dw_, db_, drm, drv, mean, inv, y, momentum, eps)
    gx = torch.empty_like(dx_)
    gw, gb = torch.empty(c, device=dev), torch.empty(c, device=dev)
    module.batch_norm_backward_train(dg_, dx_, dw_, mean, inv, gx, gw, gb)
    torch.cuda.synchronize()
    return {k: host(v) for k, v in dict(y=y, mean=mean, inv=inv, rm=drm, rv=drv, dx=gx, dw=gw,
                                        db=gb).items()}


def _check(out, x, gamma, beta, g, rm, rv, momentum=0.1, eps=1e-5):
    fy = check_batch_norm_forward(out, x, gamma, beta, rm, rv, momentum, eps)
    # the backward is checked on the device's saved statistics, as the autograd path uses them
    fb = check_batch_norm_backward(out, g, x, gamma, out["mean"], out["inv"])
    return dict(y=fy, **fb)


SHAPES = [
    (2, 3, 4, 4),      # vector path, tiny
    (5, 4, 7, 7),      # spatial 49: scalar path
    (3, 2, 1, 1),      # reference KAT shape
    (1, 3, 1, 9),      # batch 1
    (7, 16, 14, 14),   # spatial 196
    (128, 32, 14, 14), # config 5's largest BN tensor
    (4, 300, 3, 5),    # many channels, odd spatial
    (2, 1, 256, 256),  # one channel, many slices
    # one block per channel: values kept in registers (<= 8 per thread) or read twice
    (128, 96, 2, 2),
    (128, 64, 4, 4),   # exactly 2048 values per channel
    (129, 8, 4, 4),    # 2064: 1024-thread blocks (few channels), kept
    (64, 8, 7, 7),     # 3136, kept by 1024 threads
    (200, 4, 7, 7),    # 9800: 1024 threads, read twice
    (64, 130, 6, 6),   # 2304 values, 130 channels: 256 threads, read twice
]


@pytest.mark.parametrize("shape", SHAPES)
def test_batch_norm_train_matches_oracle(module, dev, shape):
    r = np.random.default_rng(hash(shape) & 0xFFFFFFFF)
    x, gamma, beta, g = _case(r, shape, 1.7, 0.3)
    c = shape[1]
    rm = r.uniform(-0.5, 0.5, c).astype(np.float32)
    rv = r.uniform(0.5, 2.0, c).astype(np.float32)
    out = _run(module, dev, x, gamma, beta, g, rm, rv)
    _check(out, x, gamma, beta, g, rm, rv)


def test_batch_norm_large_mean_small_std(module, dev):
    """|mean| / std = 1e4: the oracle's sequential fp32 sums are ill-conditioned here (its mean
    is off by many ulps, which moves x_hat by ~1e-3), so the GPU is pinned against fp64 truth
    instead: the mean is the correctly rounded fp32 of the exact mean (within 1 ulp), the
    inverse std is within 1e-6 relative, y equals the apply formula evaluated in fp64 on the
    GPU's own fp32 statistics, and the GPU mean is at least as close to the truth as the
    oracle's."""
    r = np.random.default_rng(7)
    shape = (8, 4, 16, 16)
    x, gamma, beta, g = _case(r, shape, scale=0.01, offset=100.0)
    rm, rv = np.zeros(4, np.float32), np.ones(4, np.float32)
    out = _run(module, dev, x, gamma, beta, g, rm, rv)
    x64 = x.astype(np.float64)
    mean64 = x64.mean(axis=(0, 2, 3))
    var64 = x64.var(axis=(0, 2, 3))
    ulp = np.spacing(np.abs(mean64).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(out["mean"] - mean64) <= ulp)
    np.testing.assert_allclose(out["inv"], 1 / np.sqrt(var64 + 1e-5), rtol=1e-6)
    cb = lambda v: v.astype(np.float64).reshape(1, 4, 1, 1)  # noqa: E731
    y64 = (x64 - cb(out["mean"])) * cb(out["inv"]) * cb(gamma) + cb(beta)
    np.testing.assert_allclose(out["y"], y64, rtol=1e-5, atol=2e-6)
    cpu_mean, _ = oracle.bn_batch_statistics(x, 1e-5)
    assert np.all(np.abs(out["mean"] - mean64) <= np.abs(cpu_mean - mean64) + ulp)
    n = x.size // 4
    np.testing.assert_allclose(out["rv"], 0.9 + 0.1 * var64 * n / (n - 1), rtol=1e-5)


def test_batch_norm_config2_full_shape(module, dev):
    """Config 2: [64, 128, 56, 56], x ~ N(0,1), gamma ~ U(0.5,1.5), beta ~ U(-0.1,0.1),
    g ~ N(0,1), running (0, 1), momentum 0.1, eps 1e-5."""
    r = np.random.default_rng(0x6F78696400000002)
    shape = (64, 128, 56, 56)
    x, gamma, beta, g = _case(r, shape)
    rm, rv = np.zeros(128, np.float32), np.ones(128, np.float32)
    out = _run(module, dev, x, gamma, beta, g, rm, rv)
    _check(out, x, gamma, beta, g, rm, rv)  # every element within its bound (raises otherwise)
    rep = _config2_report(out, x, gamma, beta, g, rm, rv)
    print("config 2 parity:", json.dumps(rep, sort_keys=True))
    # Measured on MI355X (deterministic: seeded inputs, fixed-order sums on both sides).  Counts
    # of elements outside max(1e-5 |cpu|, 1e-6); each of them is inside the conditioning bound
    # (worst ratio below 1).
    for k, limit in CONFIG2_OUTSIDE_STRICT.items():
        assert rep["outside_strict"][k] <= limit, (k, rep["outside_strict"][k])
    for k in ("y", "dx", "dweight", "dbias"):
        assert rep["worst_over_bound"][k] <= 1.0, k
    # against fp64 truth of the same inputs the GPU is at least as accurate as the oracle
    for k in ("mean", "inverse_std", "dweight", "dbias"):
        assert rep["max_err_vs_fp64"]["gpu"][k] <= rep["max_err_vs_fp64"]["cpu"][k], k


# Elements (of 25 690 112, or of 128 channels) outside the strict criterion at config 2, as
# measured on MI355X: every y and dx value meets max(1e-5 |cpu|, 1e-6); 46 of 128 dweight and
# 47 of 128 dbias channel sums do not, because the oracle's sequential fp32 sum of 200 704 terms
# is itself off by up to 1.5e-2 (dweight) / 8.5e-3 (dbias) against fp64 truth, where the GPU's
# fp64-accumulated sums are off by 1.1e-4 / 3.3e-5.
CONFIG2_OUTSIDE_STRICT = {"mean": 0, "inverse_std": 0, "running_mean": 0, "running_variance": 0,
                          "y": 0, "dx": 0, "dweight": 46, "dbias": 47}


def _config2_report(out, x, gamma, beta, g, rm, rv, eps=1e-5):
    """Per output: elements outside the strict criterion, the worst |gpu - cpu| over its
    conditioning bound, and each side's max error against fp64 truth of the same inputs."""
    y, mean, inv, rm1, rv1 = oracle.bn_forward(x, gamma, beta, rm, rv, True, 0.1, eps)
    dx, dw, db = oracle.bn_backward(g, x, gamma, out["mean"], out["inv"], True)
    c = x.shape[1]
    m_ = x.size // c
    cb = lambda v: np.asarray(v).reshape(1, c, 1, 1)  # noqa: E731
    x64, g64 = x.astype(np.float64), g.astype(np.float64)
    mean64 = x64.mean(axis=(0, 2, 3))
    inv64 = 1.0 / np.sqrt(x64.var(axis=(0, 2, 3)) + eps)
    xhat64 = (x64 - cb(mean64)) * cb(inv64)
    dw64 = (g64 * xhat64).sum(axis=(0, 2, 3))
    db64 = g64.sum(axis=(0, 2, 3))
    dw_cpu, db_cpu = oracle.bn_backward(g, x, gamma, mean, inv, True)[1:]
    y_terms = ((np.abs(x) + np.abs(cb(out["mean"]))) * cb(out["inv"]) * np.abs(cb(gamma))
               + np.abs(cb(beta)))
    xh = (x - cb(out["mean"])) * cb(out["inv"])
    dx_terms = np.abs(cb(gamma * out["inv"] / np.float32(m_))) * (
        m_ * np.abs(g) + np.abs(cb(db)) + np.abs(xh * cb(dw)))
    sum_abs_g = np.abs(g64).sum(axis=(0, 2, 3))
    sum_abs_gx = np.abs(g64 * xh.astype(np.float64)).sum(axis=(0, 2, 3))

    def worst(got, ref, terms):
        d = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
        return float((d / np.maximum(1e-5 * np.asarray(terms, np.float64), 1e-6)).max())

    pairs = dict(mean=(out["mean"], mean), inverse_std=(out["inv"], inv),
                 running_mean=(out["rm"], rm1), running_variance=(out["rv"], rv1),
                 y=(out["y"], y), dx=(out["dx"], dx), dweight=(out["dw"], dw),
                 dbias=(out["db"], db))
    err = lambda a, t: float(np.abs(np.asarray(a, np.float64) - t).max())  # noqa: E731
    return {
        "outside_strict": {k: int((~strict_ok(a, b)).sum()) for k, (a, b) in pairs.items()},
        "worst_over_bound": {"y": worst(out["y"], y, y_terms),
                             "dx": worst(out["dx"], dx, dx_terms),
                             "dweight": worst(out["dw"], dw, sum_abs_gx),
                             "dbias": worst(out["db"], db, sum_abs_g)},
        "max_err_vs_fp64": {
            "gpu": {"mean": err(out["mean"], mean64), "inverse_std": err(out["inv"], inv64),
                    "dweight": err(out["dw"], dw64), "dbias": err(out["db"], db64)},
            "cpu": {"mean": err(mean, mean64), "inverse_std": err(inv, inv64),
                    "dweight": err(dw_cpu, dw64), "dbias": err(db_cpu, db64)}},
    }


def test_batch_norm_reference_kats(module, dev):
    """nn.rs:761-790: running mean [0.4, 0.5] after one step, output channel mean ~0."""
    x = np.array([1, 3, 2, 4, 5, 7, 6, 8], np.float32).reshape(2, 2, 1, 2)
    ones, zeros = np.ones(2, np.float32), np.zeros(2, np.float32)
    out = _run(module, dev, x, ones, zeros, np.ones_like(x), zeros, ones)
    assert np.all(np.abs(out["rm"] - [0.4, 0.5]) < 1e-5)
    assert out["rv"][0] > 1.0
    for ch in range(2):
        assert abs(out["y"][:, ch].mean()) < 1e-5
    # jit.rs:763-782: batch statistics are recomputed on every run
    for run in ([1.0, 3.0], [10.0, 20.0]):
        x1 = np.array(run, np.float32).reshape(1, 1, 1, 2)
        o = _run(module, dev, x1, np.ones(1, np.float32), np.zeros(1, np.float32),
                 np.ones_like(x1), np.zeros(1, np.float32), np.ones(1, np.float32))
        assert np.all(np.abs(o["y"].ravel() - [-1.0, 1.0]) < 1e-4)


@pytest.mark.parametrize("shape,scale,offset", [((6, 5, 8, 8), 2.0, -0.5),
                                                ((128, 96, 2, 2), 1.0, 0.0),
                                                ((64, 128, 56, 56), 1.0, 0.0)])
def test_batch_norm_single_entry_points(module, dev, shape, scale, offset):
    """The reference's separate kernels in the reference driver's order (runtime.rs:526-669,
    1092-1156; kernel_module.rs:827-964, 1061-1092): statistics -> update_running -> apply in
    training, affine_backward -> input_backward (the affine sums as the pre-reduced sums), then
    running_inverse_std -> apply -> input_backward in eval mode.  Held to the same bars as the
    fused path: every mean / inverse std / running statistic / y / dx within max(1e-5 |cpu|,
    1e-6) or its conditioning bound, dweight / dbias within 1e-5 * sum|terms| of the oracle
    and 1e-6 * sum|terms| of fp64, the unbiased variance within max(1e-5 |v|, 1e-6) of fp64;
    at config 2's full shape and on a 2 x 2 plane (one block per channel)."""
    r = np.random.default_rng(hash(shape) & 0xFFFFF)
    n, c, h, w = shape
    m_ = n * h * w
    x, gamma, beta, g = _case(r, shape, scale, offset)
    rm, rv = r.uniform(-1, 1, c).astype(np.float32), r.uniform(0.5, 2, c).astype(np.float32)
    dx_, dgam, dbet, dg_ = (to_dev(a, dev) for a in (x, gamma, beta, g))
    mean, inv, unb = (torch.empty(c, device=dev) for _ in range(3))
    module.batch_norm_statistics(n, c, h * w, 1e-5, dx_, mean, inv, unb)
    rm0, rv0 = to_dev(rm, dev), to_dev(rv, dev)
    rm1, rv1 = torch.empty_like(rm0), torch.empty_like(rv0)
    module.batch_norm_update_running(0.1, mean, unb, rm0, rv0, rm1, rv1)
    y = torch.empty_like(dx_)
    module.batch_norm_apply(c, h * w, dx_, dgam, dbet, mean, inv, y)
    gw, gb = torch.empty(c, device=dev), torch.empty(c, device=dev)
    module.batch_norm_affine_backward(n, c, h * w, dg_, dx_, mean, inv, gw, gb)
    gx = torch.empty_like(dx_)
    module.batch_norm_input_backward(c, h * w, m_, True, dg_, dx_, dgam, mean, inv, gw, gb, gx)
    torch.cuda.synchronize()
    out = dict(y=host(y), mean=host(mean), inv=host(inv), rm=host(rm1), rv=host(rv1),
               dx=host(gx), dw=host(gw), db=host(gb))
    check_batch_norm_forward(out, x, gamma, beta, rm, rv)
    check_batch_norm_backward(out, g, x, gamma, out["mean"], out["inv"])
    # the unbiased variance the update consumes: sum (x - mean)^2 / (M - 1), against fp64
    var64 = x.astype(np.float64).var(axis=(0, 2, 3))
    assert_close(host(unb), var64 * m_ / (m_ - 1), what="unbiased variance vs fp64")
    del y, gx
    # eval mode: running inverse std, apply with the running statistics, dx = g * w * inv
    rinv = torch.empty(c, device=dev)
    module.batch_norm_running_inverse_std(1e-5, rv0, rinv)
    ye, gxe = torch.empty_like(dx_), torch.empty_like(dx_)
    module.batch_norm_apply(c, h * w, dx_, dgam, dbet, rm0, rinv, ye)
    module.batch_norm_input_backward(c, h * w, m_, False, dg_, dx_, dgam, rm0, rinv, gw, gb,
                                     gxe)
    torch.cuda.synchronize()
    rinv_h = host(rinv)
    assert_close(rinv_h, 1.0 / np.sqrt(rv + np.float32(1e-5)), what="running inverse std")
    y_eval, *_ = oracle.bn_forward(x, gamma, beta, rm, rv, False)
    cb = lambda v: v.reshape(1, c, 1, 1)  # noqa: E731
    ye_h = host(ye)
    if not strict_ok(ye_h, y_eval).all():  # x - running mean cancels: conditioning bound
        terms = (np.abs(x) + np.abs(cb(rm))) * cb(rinv_h) * np.abs(cb(gamma)) + np.abs(cb(beta))
        assert_within(ye_h, y_eval, np.maximum(1e-5 * terms, 1e-6), "eval apply")
    dx_eval, _, _ = oracle.bn_backward(g, x, gamma, rm, rinv_h, False)
    assert_close(host(gxe), dx_eval, what="eval input backward")


def test_batch_norm_workspace_reuse_and_repeat(module, dev):
    """The reduction counters reset themselves: repeated calls give identical results."""
    r = np.random.default_rng(3)
    x, gamma, beta, g = _case(r, (16, 24, 10, 12))
    rm, rv = np.zeros(24, np.float32), np.ones(24, np.float32)
    first = _run(module, dev, x, gamma, beta, g, rm, rv)
    for _ in range(3):
        again = _run(module, dev, x, gamma, beta, g, rm, rv)
        for k in first:
            assert np.array_equal(first[k], again[k]), k


@pytest.mark.parametrize("shape", [(2, 3, 4, 4), (5, 4, 7, 7), (128, 96, 2, 2), (128, 1280, 1, 1),
                                   (64, 32, 4, 4), (7, 16, 14, 14), (128, 32, 14, 14),
                                   (3, 5, 3, 3), (64, 8, 7, 7), (128, 4, 4, 4)])
def test_batch_norm_relu_fused_matches_unfused(module, dev, shape):
    """ConvNormAct's BN + ReLU in one launch per direction: the fused forward equals the ReLU
    kernel applied to the unfused forward, and the fused backward equals the unfused backward
    fed the ReLU backward kernel's gradient -- bit for bit (same sums, same element formulas),
    on the one-block-per-channel path (small planes) and the reduce + map path (14 x 14);
    the unfused BN itself is pinned to the oracle."""
    r = np.random.default_rng(hash(shape) & 0xFFFF)
    x, gamma, beta, g = _case(r, shape, 1.3, 0.2)
    c = shape[1]
    rm = r.uniform(-0.5, 0.5, c).astype(np.float32)
    rv = r.uniform(0.5, 2.0, c).astype(np.float32)
    dx_, dw_, db_, dg_ = to_dev(x, dev), to_dev(gamma, dev), to_dev(beta, dev), to_dev(g, dev)

    def stats():
        return (to_dev(rm, dev), to_dev(rv, dev), torch.empty(c, device=dev),
                torch.empty(c, device=dev))

    # unfused: BN forward, ReLU, ReLU backward, BN backward
    rm1, rv1, m1, i1 = stats()
    y_bn = torch.empty_like(dx_)
    module.batch_norm_forward_train(dx_, dw_, db_, rm1, rv1, m1, i1, y_bn, 0.1, 1e-5)
    y1 = torch.empty_like(dx_)
    module.relu(y_bn, y1)
    g_masked = torch.empty_like(dx_)
    module.relu_backward(dg_, y_bn, g_masked)
    gx1, gw1, gb1 = torch.empty_like(dx_), torch.empty(c, device=dev), torch.empty(c, device=dev)
    module.batch_norm_backward_train(g_masked, dx_, dw_, m1, i1, gx1, gw1, gb1)
    # fused
    rm2, rv2, m2, i2 = stats()
    y2 = torch.empty_like(dx_)
    module.batch_norm_relu_forward_train(dx_, dw_, db_, rm2, rv2, m2, i2, y2, 0.1, 1e-5)
    gx2, gw2, gb2 = torch.empty_like(dx_), torch.empty(c, device=dev), torch.empty(c, device=dev)
    module.batch_norm_relu_backward_train(dg_, y2, dx_, dw_, m2, i2, gx2, gw2, gb2)
    torch.cuda.synchronize()
    for a, b, what in ((y2, y1, "y"), (m2, m1, "mean"), (i2, i1, "inv"), (rm2, rm1, "rm"),
                       (rv2, rv1, "rv"), (gx2, gx1, "dx"), (gw2, gw1, "dw"), (gb2, gb1, "db")):
        np.testing.assert_array_equal(host(a), host(b), err_msg=what)
    assert (host(y2) >= 0).all()
    # the unfused composition against the oracle
    out = dict(y=host(y_bn), mean=host(m1), inv=host(i1), rm=host(rm1), rv=host(rv1))
    check_batch_norm_forward(out, x, gamma, beta, rm, rv)
    gm = oracle.relu_backward(g, host(y_bn))
    np.testing.assert_array_equal(host(g_masked), gm)
    check_batch_norm_backward(dict(dx=host(gx1), dw=host(gw1), db=host(gb1)), gm, x, gamma,
                              host(m1), host(i1))


@pytest.mark.parametrize("shape", [(2, 3, 4, 4), (128, 96, 2, 2), (128, 1280, 1, 1),
                                   (128, 32, 14, 14), (3, 5, 3, 3), (64, 8, 7, 7)])
@pytest.mark.parametrize("relu", [False, True])
def test_conv_batch_norm_backward_writes_conv_bias(module, dev, shape, relu):
    """The BatchNorm backward that also reduces its input gradient per channel (the bias
    gradient of the convolution feeding it): BatchNorm outputs bit-equal to the plain entry
    point's, on the one-block-per-channel path and the reduce + map path (14 x 14); the
    convolution bias gradient against the oracle's conv2d bias sum over that input gradient
    (|d| <= 1e-5 * sum|terms|: fp64 block sums against the CPU's fp32 running sum)."""
    r = np.random.default_rng(hash((shape, relu)) & 0xFFFF)
    x, gamma, beta, g = _case(r, shape, 1.3, 0.2)
    c = shape[1]
    dx_, dw_, dg_ = to_dev(x, dev), to_dev(gamma, dev), to_dev(g, dev)
    mean = to_dev(r.standard_normal(c).astype(np.float32) * 0.1, dev)
    inv = to_dev(r.uniform(0.5, 2.0, c).astype(np.float32), dev)
    y = to_dev(np.maximum(r.standard_normal(shape).astype(np.float32), 0), dev) if relu else None

    def outs():
        return (torch.empty_like(dx_), torch.empty(c, device=dev), torch.empty(c, device=dev))

    gx1, gw1, gb1 = outs()
    if relu:
        module.batch_norm_relu_backward_train(dg_, y, dx_, dw_, mean, inv, gx1, gw1, gb1)
    else:
        module.batch_norm_backward_train(dg_, dx_, dw_, mean, inv, gx1, gw1, gb1)
    gx2, gw2, gb2 = outs()
    conv_bias = torch.full((c,), float("nan"), device=dev)
    module.conv_batch_norm_backward_train(dg_, y, dx_, dw_, mean, inv, gx2, gw2, gb2, conv_bias)
    torch.cuda.synchronize()
    for a, b, what in ((gx2, gx1, "dx"), (gw2, gw1, "dw"), (gb2, gb1, "db")):
        np.testing.assert_array_equal(host(a), host(b), err_msg=what)
    dx = host(gx2)
    assert_within(host(conv_bias), oracle.conv2d_bias_backward(dx),
                  1e-5 * np.abs(dx).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-7, "conv bias")
    with pytest.raises(ox.OxideError) as e:
        module.conv_batch_norm_backward_train(dg_, y, dx_, dw_, mean, inv, gx2, gw2, gb2, None)
    assert e.value.status == ox.INVALID_SHAPE


@pytest.mark.parametrize("shape", [(128, 96, 2, 2), (128, 128, 1, 1), (64, 8, 7, 7),
                                   (7, 16, 14, 14), (3, 5, 3, 3)])
def test_batch_norm_add_fused_matches_unfused(module, dev, shape):
    """BatchNorm forward + residual add in one pass: the output equals the add kernel applied to
    the plain forward's output bit for bit, with identical statistics, on the
    one-block-per-channel path (values kept or read twice) and the reduce + map path."""
    r = np.random.default_rng(hash(shape) & 0xFFFF)
    x, gamma, beta, _ = _case(r, shape, 1.1, 0.4)
    c = shape[1]
    skip = r.standard_normal(shape).astype(np.float32)
    rm = r.uniform(-0.5, 0.5, c).astype(np.float32)
    rv = r.uniform(0.5, 2.0, c).astype(np.float32)
    dx_, dw_, db_, ds_ = to_dev(x, dev), to_dev(gamma, dev), to_dev(beta, dev), to_dev(skip, dev)

    def stats():
        return (to_dev(rm, dev), to_dev(rv, dev), torch.empty(c, device=dev),
                torch.empty(c, device=dev))

    rm1, rv1, m1, i1 = stats()
    y = torch.empty_like(dx_)
    module.batch_norm_forward_train(dx_, dw_, db_, rm1, rv1, m1, i1, y, 0.1, 1e-5)
    unfused = torch.empty_like(dx_)
    module.add(y, ds_, unfused)
    rm2, rv2, m2, i2 = stats()
    fused = torch.empty_like(dx_)
    module.batch_norm_add_forward_train(dx_, dw_, db_, rm2, rv2, m2, i2, ds_, fused)
    torch.cuda.synchronize()
    for a, b, what in ((fused, unfused, "y + skip"), (m2, m1, "mean"), (i2, i1, "inv"),
                       (rm2, rm1, "running mean"), (rv2, rv1, "running variance")):
        np.testing.assert_array_equal(host(a), host(b), err_msg=what)
    check_batch_norm_forward(dict(y=host(y), mean=host(m1), inv=host(i1), rm=host(rm1),
                                  rv=host(rv1)), x, gamma, beta, rm, rv)
    with pytest.raises(ox.OxideError):
        module.batch_norm_add_forward_train(dx_, dw_, db_, rm2, rv2, m2, i2, fused, fused)
