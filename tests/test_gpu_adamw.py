"""Fused AdamW on the GPU, bit-exact against the oracle's restatement of optim.rs:98-125,
including config 4's full 64M-element step at t=10, in-place and out-of-place outputs, ragged
and unaligned sizes, and the multi-tensor launch."""

import numpy as np
import pytest
import torch

import oracle
import oxide_hip as ox
from helpers import assert_bitexact, host, to_dev

pytestmark = pytest.mark.gpu

LR, WD, B1, B2, EPS = 1e-3, 0.01, 0.9, 0.999, 1e-8


def _state(r, n):
    p = (r.standard_normal(n) * 0.02).astype(np.float32)
    g = (r.standard_normal(n) * 1e-3).astype(np.float32)
    gp = (r.standard_normal(n) * 1e-3).astype(np.float32)
    m = ((1 - 0.9) * gp).astype(np.float32)
    v = ((1 - 0.999) * gp * gp).astype(np.float32)
    return p, g, m, v


@pytest.mark.parametrize("n", [1, 5, 4096, 4099, 1 << 20, 64 << 20])
@pytest.mark.parametrize("step", [10])
def test_adamw_bitexact(module, dev, n, step):
    r = np.random.default_rng(0x6F78696400000004)
    p, g, m, v = _state(r, n)
    p_ref, m_ref, v_ref = oracle.adamw_update(p, g, m, v, step, LR, WD, B1, B2, EPS)
    c1, c2 = ox.adamw_corrections(B1, B2, step)
    dp, dg, dm, dv = (to_dev(x, dev) for x in (p, g, m, v))
    module.adamw(LR, WD, B1, B2, c1, c2, EPS, dp, dg, dm, dv, dp, dm, dv)  # in place
    torch.cuda.synchronize()
    assert_bitexact(host(dp), p_ref, "param")
    assert_bitexact(host(dm), m_ref, "m")
    assert_bitexact(host(dv), v_ref, "v")


def test_adamw_out_of_place_and_steps(module, dev, rng):
    n = 10007
    p, g, m, v = _state(rng, n)
    dp, dg, dm, dv = (to_dev(x, dev) for x in (p, g, m, v))
    po, mo, vo = (torch.empty_like(dp) for _ in range(3))
    for step in (1, 2, 3, 50, 1000):
        c1, c2 = ox.adamw_corrections(B1, B2, step)
        module.adamw(LR, WD, B1, B2, c1, c2, EPS, dp, dg, dm, dv, po, mo, vo)
        torch.cuda.synchronize()
        p, m, v = oracle.adamw_update(p, g, m, v, step, LR, WD, B1, B2, EPS)
        assert_bitexact(host(po), p, f"param step {step}")
        assert_bitexact(host(mo), m, f"m step {step}")
        assert_bitexact(host(vo), v, f"v step {step}")
        dp.copy_(po)
        dm.copy_(mo)
        dv.copy_(vo)
    # inputs are untouched by an out-of-place update
    assert_bitexact(host(dg), g, "grad untouched")


def test_adamw_unaligned_view(module, dev, rng):
    n = 999
    p, g, m, v = _state(rng, n)
    bufs = []
    for x in (p, g, m, v):
        t = torch.zeros(n + 1, device=dev)
        t[1:] = to_dev(x, dev)
        bufs.append(t[1:])
    c1, c2 = ox.adamw_corrections(B1, B2, 3)
    module.adamw(LR, WD, B1, B2, c1, c2, EPS, *bufs, bufs[0], bufs[2], bufs[3])
    torch.cuda.synchronize()
    p_ref, m_ref, v_ref = oracle.adamw_update(p, g, m, v, 3, LR, WD, B1, B2, EPS)
    assert_bitexact(host(bufs[0]), p_ref, "unaligned param")
    assert_bitexact(host(bufs[2]), m_ref, "unaligned m")


def test_adamw_multi_tensor_matches_per_tensor(module, dev, rng):
    """One launch over many tensors (config 5 updates 186 parameter tensors per step)."""
    sizes = [1, 3, 16, 100, 4096, 9, 65537, 288, 1152, 7] * 12  # 120 tensors -> 3 launches
    tensors, refs = [], []
    for n in sizes:
        p, g, m, v = _state(rng, n)
        refs.append(oracle.adamw_update(p, g, m, v, 7, LR, 1e-4, B1, B2, EPS))
        tensors.append(tuple(to_dev(x, dev) for x in (p, g, m, v)))
    c1, c2 = ox.adamw_corrections(B1, B2, 7)
    module.adamw_multi_tensor(LR, 1e-4, B1, B2, c1, c2, EPS, tensors)
    torch.cuda.synchronize()
    for i, ((dp, _, dm, dv), (p_ref, m_ref, v_ref)) in enumerate(zip(tensors, refs)):
        assert_bitexact(host(dp), p_ref, f"tensor {i} param")
        assert_bitexact(host(dm), m_ref, f"tensor {i} m")
        assert_bitexact(host(dv), v_ref, f"tensor {i} v")


def test_adamw_first_step_closed_form(module, dev, rng):
    """t=1 from zero moments: p1 = p0 - lr * (g / (|g| + eps) + wd * p0) in exact arithmetic."""
    n = 4096
    p = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    dp, dg = to_dev(p, dev), to_dev(g, dev)
    dm, dv = torch.zeros_like(dp), torch.zeros_like(dp)
    c1, c2 = ox.adamw_corrections(B1, B2, 1)
    module.adamw(1e-2, 0.1, B1, B2, c1, c2, EPS, dp, dg, dm, dv, dp, dm, dv)
    torch.cuda.synchronize()
    expect = p.astype(np.float64) - 1e-2 * (np.sign(g) + 0.1 * p.astype(np.float64))
    np.testing.assert_allclose(host(dp), expect, rtol=1e-5, atol=1e-6)


CONFIG5_SIZES = [864, 32, 32, 32, 288, 32, 1024, 32, 32, 32] * 18 + [12800, 10, 1280, 10, 5, 7]


@pytest.mark.parametrize("table", ["config5", "block", "many"])
def test_adamw_table_step_matches_multi_tensor_step(module, dev, rng, table):
    """The one-launch device-table update equals the step-counting multi-tensor update bit for
    bit over three steps: 186 tensors as in config 5 (more than one 48-tensor launch of the
    latter) and 256 tensors of 1 to 5000 values (each block's tensor found by one thread per
    tensor), and 700 such tensors (the chunk search then takes two rounds of the block's 256
    probes); the step counter advances once per call."""
    if table == "config5":
        sizes = CONFIG5_SIZES
        assert len(sizes) == 186
    else:
        sizes = [int(v) for v in rng.integers(1, 5001, 256 if table == "block" else 700)]
    state = [_state(rng, n) for n in sizes]
    a = [tuple(to_dev(x, dev) for x in s) for s in state]
    b = [tuple(to_dev(x, dev) for x in s) for s in state]
    step_a = torch.zeros(1, dtype=torch.int32, device=dev)
    step_b = torch.zeros(1, dtype=torch.int32, device=dev)
    for _ in range(3):
        module.adamw_multi_tensor_step(LR, 1e-4, B1, B2, EPS, step_a, a)
        keep = module.adamw_table_step(LR, 1e-4, B1, B2, EPS, step_b, b)
        torch.cuda.synchronize()
        del keep
    assert int(host(step_a)[0]) == int(host(step_b)[0]) == 3
    for i, (ta, tb) in enumerate(zip(a, b)):
        for k, what in ((0, "param"), (2, "m"), (3, "v")):
            assert_bitexact(host(tb[k]), host(ta[k]), f"tensor {i} {what}")
