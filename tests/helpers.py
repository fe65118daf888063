"""Comparison helpers shared by the parity tests."""

import numpy as np


def to_dev(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
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
