"""Elementwise add / mul / relu, their backward, accumulate and the fused chain on the GPU,
bit-exact against the oracle (evaluation.rs:21-34, autograd.rs:94-147).  Sizes cover empty,
ragged (n % 4 != 0), unaligned views and config 1's full [4096, 4096]."""

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_bitexact, host, to_dev

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 4, 5, 1023, 4099, 65536 + 7, 1 << 20]


def _inputs(rng, n):
    return [rng.uniform(-1, 1, n).astype(np.float32) for _ in range(3)]


@pytest.mark.parametrize("n", SIZES)
def test_binary_and_unary_ops_bitexact(module, dev, rng, n):
    a, b, c = _inputs(rng, n)
    da, db, dc = to_dev(a, dev), to_dev(b, dev), to_dev(c, dev)
    out = torch.empty_like(da)
    cases = [
        (module.add, (da, db), oracle.add(a, b)),
        (module.mul, (da, db), oracle.mul(a, b)),
        (module.relu, (da,), oracle.relu(a)),
        (module.mul_backward, (db, dc), oracle.mul_backward(b, c)),
        (module.relu_backward, (db, da), oracle.relu_backward(b, a)),
        (module.accumulate, (da, db), oracle.accumulate(a, b)),
    ]
    for fn, args, ref in cases:
        out.fill_(np.nan)
        fn(*args, out)
        torch.cuda.synchronize()
        assert_bitexact(host(out), ref, fn.__name__)


def test_in_place_and_unaligned(module, dev, rng):
    a, b, _ = _inputs(rng, 10001)
    da, db = to_dev(a, dev), to_dev(b, dev)
    module.add(da, db, da)  # in place: output == input
    torch.cuda.synchronize()
    assert_bitexact(host(da), oracle.add(a, b), "in-place add")
    # views offset by one float are only 4-byte aligned: the scalar path runs
    big = to_dev(np.concatenate([[0.0], a]).astype(np.float32), dev)
    view = big[1:]
    out = torch.empty(10002, device=dev)[1:]
    module.relu(view, out)
    torch.cuda.synchronize()
    assert_bitexact(host(out), oracle.relu(a), "unaligned relu")


def test_special_values(module, dev):
    x = np.array([np.nan, -0.0, 0.0, -np.inf, np.inf, 1e-45, -1e-45, 3.4e38], np.float32)
    g = np.arange(1, 9, dtype=np.float32)
    dx, dg = to_dev(x, dev), to_dev(g, dev)
    out = torch.empty_like(dx)
    module.relu(dx, out)
    torch.cuda.synchronize()
    assert_bitexact(host(out), oracle.relu(x), "relu special")
    assert np.all(np.signbit(host(out)) == False)  # noqa: E712  (x > 0 ? x : 0 gives +0)
    module.relu_backward(dg, dx, out)
    torch.cuda.synchronize()
    assert_bitexact(host(out), oracle.relu_backward(g, x), "relu_backward special")


def test_empty_is_noop(module, dev):
    e = torch.empty(0, device=dev)
    module.add(e, e, e)
    module.relu(e, e)
    torch.cuda.synchronize()


@pytest.mark.parametrize("n", [7, 4096 * 4096])
def test_chain_forward_backward_config1(module, dev, n):
    """Config 1: relu((a+b)*c) at [4096, 4096] and backward of sum() (upstream ones), both as
    the fused kernels and as the reference's op-by-op sequence."""
    r = np.random.default_rng(0x6F78696400000001)
    a, b, c = (r.uniform(-1, 1, n).astype(np.float32) for _ in range(3))
    da, db, dc = to_dev(a, dev), to_dev(b, dev), to_dev(c, dev)
    y = torch.empty_like(da)
    module.elementwise_chain_forward(da, db, dc, y)
    ga, gb, gc = torch.empty_like(da), torch.empty_like(da), torch.empty_like(da)
    module.elementwise_chain_backward(da, db, dc, None, ga, gb, gc)
    torch.cuda.synchronize()
    y_ref = oracle.chain_forward(a, b, c)
    ra, rb, rc = oracle.chain_backward_ones(a, b, c)
    assert_bitexact(host(y), y_ref, "chain forward")
    assert_bitexact(host(ga), ra, "chain da")
    assert_bitexact(host(gb), rb, "chain db")
    assert_bitexact(host(gc), rc, "chain dc")
    # op-by-op (add -> mul -> relu, then relu_backward / mul_backward) gives the same bits
    s, m, yy = torch.empty_like(da), torch.empty_like(da), torch.empty_like(da)
    module.add(da, db, s)
    module.mul(s, dc, m)
    module.relu(m, yy)
    ones = torch.ones_like(da)
    gm, gl, gr = torch.empty_like(da), torch.empty_like(da), torch.empty_like(da)
    module.relu_backward(ones, m, gm)
    module.mul_backward(gm, dc, gl)
    module.mul_backward(gm, s, gr)
    torch.cuda.synchronize()
    assert_bitexact(host(yy), y_ref, "op-by-op forward")
    assert_bitexact(host(gl), ra, "op-by-op da")
    assert_bitexact(host(gr), rc, "op-by-op dc")
    # explicit upstream gradient
    g = r.standard_normal(n).astype(np.float32)
    module.elementwise_chain_backward(da, db, dc, to_dev(g, dev), ga, gb, gc)
    torch.cuda.synchronize()
    on = oracle.relu_backward(g, oracle.mul(oracle.add(a, b), c))
    assert_bitexact(host(ga), oracle.mul_backward(on, c), "chain da (g)")
    assert_bitexact(host(gc), oracle.mul_backward(on, oracle.add(a, b)), "chain dc (g)")


def test_argmax_last_index_wins_ties(module, dev, rng):
    """mnist_training.rs:201-218 (max_by(total_cmp): the last maximum wins)."""
    rows = np.array([[1, 3, 3, 2], [0, -0.0, 0.0, -1], [5, 5, 5, 5], [np.nan, 1, 2, 3],
                     [-np.inf, -np.inf, -np.inf, -np.inf]], np.float32)
    logits = np.concatenate([rows, rng.integers(-3, 3, (251, 4)).astype(np.float32)])
    big = rng.integers(-5, 5, (33, 1000)).astype(np.float32)
    for arr in (logits, big):
        d = to_dev(arr, dev)
        idx = torch.empty(arr.shape[0], dtype=torch.int32, device=dev)
        module.argmax_rows(d, idx)
        torch.cuda.synchronize()
        assert np.array_equal(host(idx).astype(np.uint64), oracle.argmax_rows(arr))
