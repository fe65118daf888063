"""Comparison helpers shared by the parity tests."""

import numpy as np


def to_dev(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    """Host copy of a torch tensor or of a library-owned device view."""
    if hasattr(t, "host"):
        return t.host()
    return t.detach().cpu().numpy()


def assert_bitexact(got, ref, what=""):
    """Bit-exact fp32 comparison with +0 and -0 treated as equal and NaN equal to NaN."""
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    if not same.all():
        idx = np.flatnonzero(~same.ravel())[:5]
        raise AssertionError(f"{what}: {(~same).sum()} of {same.size} differ; first at {idx}: "
                             f"got {got.ravel()[idx]} ref {ref.ravel()[idx]}")


def strict_ok(got, ref, rtol=1e-5, atol=1e-6):
    """The north-star criterion per element: |got - ref| <= max(rtol * |ref|, atol)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return np.abs(got - ref) <= np.maximum(rtol * np.abs(ref), atol)


def assert_close(got, ref, rtol=1e-5, atol=1e-6, what=""):
    ok = strict_ok(got, ref, rtol, atol)
    if not ok.all():
        g = np.asarray(got, np.float64).ravel()
        r = np.asarray(ref, np.float64).ravel()
        bad = np.flatnonzero(~ok.ravel())
        worst = bad[np.argmax(np.abs(g[bad] - r[bad]))]
        raise AssertionError(f"{what}: {bad.size} of {ok.size} outside rtol={rtol} atol={atol};"
                             f" worst at {worst}: got {g[worst]!r} ref {r[worst]!r}")


def assert_conv_forward(got, x, weight, bias, stride, padding, groups, what=""):
    """A conv2d forward against the oracle: bit-exact where the library sums in the CPU path's
    order (oxh_conv2d_forward_serial), else (four ordered parts over the input channels) within
    1e-5 * sum|terms| (the terms' magnitudes through the oracle)."""
    import oracle
    import oxide_hip as ox

    ref = oracle.conv2d_forward(x, weight, bias, stride, padding, groups)
    n, cin, h, w = x.shape
    cout, _, k, _ = weight.shape
    if ox.conv2d_forward_serial(ox.conv2d_shape(n, cin, h, w, cout, k, stride, padding, groups)):
        assert_bitexact(got, ref, what)
    else:
        mag = oracle.conv2d_forward(np.abs(x), np.abs(weight), np.abs(bias), stride, padding,
                                    groups)
        assert_within(got, ref, 1e-5 * mag.astype(np.float64) + 1e-7, what)


def assert_conv_input_gradient(got, gradient, weight, stride, padding, groups, input_shape,
                               addend=None, what=""):
    """A conv2d input gradient (+ addend) against the oracle: bit-exact where the library sums
    in the CPU path's order (oxh_conv2d_input_backward_serial), else (four ordered parts over
    the output channels) within 1e-5 * sum|terms| (+ one rounding of the addend's add)."""
    import oracle
    import oxide_hip as ox

    zeros = np.zeros(input_shape, np.float32)
    ref = oracle.conv2d_backward(gradient, zeros, weight, stride, padding, groups)[0]
    if addend is not None:
        ref = oracle.accumulate(addend, ref)
    n, cin, h, w = input_shape
    cout, _, k, _ = weight.shape
    if ox.conv2d_input_backward_serial(ox.conv2d_shape(n, cin, h, w, cout, k, stride, padding,
                                                       groups)):
        assert_bitexact(got, ref, what)
    else:
        mag = oracle.conv2d_backward(np.abs(gradient), zeros, np.abs(weight), stride, padding,
                                     groups)[0].astype(np.float64)
        bound = 1e-5 * mag + 1e-7
        if addend is not None:
            bound = bound + np.abs(np.asarray(ref, np.float64)) * 2.0 ** -23
        assert_within(got, ref, bound, what)


def assert_within(got, ref, bound, what=""):
    """|got - ref| <= bound elementwise (bound: a conditioning-aware error bound)."""
    d = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
    bound = np.broadcast_to(np.asarray(bound, np.float64), d.shape)
    ok = d <= bound
    if not ok.all():
        bad = np.flatnonzero(~ok.ravel())
        worst = bad[np.argmax((d.ravel() / np.maximum(bound.ravel(), 1e-300))[bad])]
        raise AssertionError(f"{what}: {bad.size} of {ok.size} outside the bound; worst at "
                             f"{worst}: |d|={d.ravel()[worst]!r} bound={bound.ravel()[worst]!r}")


def check_batch_norm_forward(out, x, gamma, beta, rm, rv, momentum=0.1, eps=1e-5, relu=False):
    """out: dict with y, mean, inv, rm, rv from the device for inputs x, gamma, beta and running
    statistics rm, rv (before the update); relu: y is relu(batch norm) (ReLU is 1-Lipschitz, so
    the batch-norm bound carries over).  Returns the fraction of y within the strict
    criterion."""
    import oracle

    y, mean, inv, rm1, rv1 = oracle.bn_forward(x, gamma, beta, rm, rv, True, momentum, eps)
    if relu:
        y = oracle.relu(y)
    c = x.shape[1]
    assert_close(out["mean"], mean, what="mean")
    assert_close(out["inv"], inv, what="inverse std")
    assert_close(out["rm"], rm1, what="running mean")
    assert_close(out["rv"], rv1, what="running var")
    cb = lambda v: v.reshape(1, c, 1, 1)  # noqa: E731
    # y = ((x - mean) * inv) * w + b: x - mean cancels, so the terms are x * inv * w,
    # mean * inv * w and b (one ulp of the mean moves y by |mean| * inv * |w| * 2^-24)
    y_terms = ((np.abs(x) + np.abs(cb(mean))) * cb(inv) * np.abs(cb(gamma))
               + np.abs(cb(beta)))
    ok = strict_ok(out["y"], y)
    if not ok.all():
        assert_within(out["y"], y, np.maximum(1e-5 * y_terms, 1e-6), "y")
    return ok.mean()


def check_batch_norm_backward(out, g, x, gamma, mean, inv):
    """out: dict with dx, dw, db from the device for upstream gradient g and the saved batch
    statistics (mean, inv) the device used.  Returns the strict-criterion fractions."""
    import oracle

    dx, dw, db = oracle.bn_backward(g, x, gamma, mean, inv, True)
    n, c, h, w = x.shape
    cb = lambda v: v.reshape(1, c, 1, 1)  # noqa: E731
    # dx terms: (w*inv/M) * (M*g, sum g, x_hat * sum g x_hat)
    m_ = n * h * w
    xhat = (x - cb(mean)) * cb(inv)
    coef = np.abs(cb(gamma * inv / np.float32(m_)))
    dx_terms = coef * (m_ * np.abs(g) + np.abs(cb(db)) + np.abs(xhat * cb(dw)))
    ok = strict_ok(out["dx"], dx)
    if not ok.all():
        assert_within(out["dx"], dx, np.maximum(1e-5 * dx_terms, 1e-6), "dx")
    # channel sums: conditioning bound vs the oracle and a tight bound vs fp64 of the same terms
    sum_abs_g = np.abs(g.astype(np.float64)).sum(axis=(0, 2, 3))
    gx32 = (g * ((x - cb(mean)) * cb(inv))).astype(np.float32)
    sum_abs_gx = np.abs(gx32.astype(np.float64)).sum(axis=(0, 2, 3))
    assert_within(out["db"], db, 1e-5 * sum_abs_g + 1e-6, "dbias vs oracle")
    assert_within(out["dw"], dw, 1e-5 * sum_abs_gx + 1e-6, "dweight vs oracle")
    assert_within(out["db"], g.astype(np.float64).sum(axis=(0, 2, 3)),
                  1e-6 * sum_abs_g + 1e-7, "dbias vs fp64")
    assert_within(out["dw"], gx32.astype(np.float64).sum(axis=(0, 2, 3)),
                  1e-6 * sum_abs_gx + 1e-7, "dweight vs fp64")
    return dict(dx=ok.mean(), dw=strict_ok(out["dw"], dw).mean(),
                db=strict_ok(out["db"], db).mean())
