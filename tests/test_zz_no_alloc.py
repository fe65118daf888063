"""The allocation-free BatchNorm2d training forward (oxh_batch_norm_forward_train_no_alloc,
partials in a static per-GPU array) against oxh_batch_norm_forward_train with a caller
workspace, through the C ABI: bit-identical outputs, saved statistics and running statistics
on two calls in a row, the second on a smaller input, in both the reduce + apply path and the
one-block-per-channel path; shapes beyond the static array are rejected before any launch."""

import ctypes

import numpy as np
import pytest
import torch

import oxide_hip as ox
from helpers import assert_bitexact, host, to_dev

pytestmark = pytest.mark.gpu


def _inputs(r, shape):
    n, c, h, w = shape
    x = (r.standard_normal(shape) * 1.3 + 0.2).astype(np.float32)
    gamma = r.uniform(0.5, 1.5, c).astype(np.float32)
    beta = r.uniform(-0.1, 0.1, c).astype(np.float32)
    rm = r.uniform(-0.5, 0.5, c).astype(np.float32)
    rv = r.uniform(0.5, 2.0, c).astype(np.float32)
    return x, gamma, beta, rm, rv


def _forward(dev, arrays, no_alloc):
    x, gamma, beta, rm, rv = (to_dev(a, dev) for a in arrays)
    n, c, h, w = x.shape
    y = torch.empty_like(x)
    mean, inv = torch.empty(c, device=dev), torch.empty(c, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    if no_alloc:
        st = ox.lib().oxh_batch_norm_forward_train_no_alloc(
            s, n, c, h * w, 0.1, 1e-5, p(x), p(gamma), p(beta), p(rm), p(rv), p(mean), p(inv),
            p(y))
        keep = None
    else:
        size = ox.batch_norm_workspace_size(n, c, h * w)
        keep = torch.empty(size // 4, dtype=torch.float32, device=dev)
        st = ox.lib().oxh_batch_norm_forward_train(
            s, n, c, h * w, 0.1, 1e-5, p(x), p(gamma), p(beta), p(rm), p(rv), p(mean), p(inv),
            p(y), p(keep), size)
    assert st == ox.OK, ox.lib().oxh_last_error()
    torch.cuda.synchronize()
    del keep
    return {k: host(v) for k, v in dict(y=y, mean=mean, inv=inv, rm=rm, rv=rv).items()}


@pytest.mark.parametrize("shapes", [
    [(16, 64, 28, 28), (2, 8, 16, 16)],   # reduce + apply path (partials in the array)
    [(64, 128, 56, 56), (8, 32, 12, 12)],  # config 2, then a smaller tensor
    [(128, 96, 2, 2), (32, 16, 4, 4)],     # one block per channel
])
def test_no_alloc_forward_equals_workspace_forward(dev, shapes):
    ox.init(0)
    r = np.random.default_rng(0x6E6F616C)
    for shape in shapes:
        print("no-alloc BN forward", shape, flush=True)
        arrays = _inputs(r, shape)
        ref = _forward(dev, arrays, False)
        got = _forward(dev, arrays, True)
        for k in ref:
            assert_bitexact(got[k], ref[k], f"{shape} {k}")


def test_no_alloc_array_covers_every_accepted_shape():
    """The static array holds the partials of the largest shape the batch-norm entry points
    accept (65 535 channels, one 16-byte partial each); more channels are refused on the host
    before any launch."""
    assert ox.batch_norm_workspace_size(2, 65535, 4) <= 1 << 20
    assert ox.batch_norm_workspace_size(64, 2048, 3136) <= 1 << 20
    lib = ox.lib()
    st = lib.oxh_batch_norm_forward_train_no_alloc(None, 2, 65536, 4, 0.1, 1e-5, None, None,
                                                   None, None, None, None, None, None)
    assert st == ox.INVALID_SHAPE
    assert b"channels" in lib.oxh_last_error()
