"""Pins of the two xorshift64 streams the oracle restates: the deterministic weight init
(crates/oxide-torch/src/nn.rs:657-674) and the MNIST batch shuffle
(crates/oxide-torch/src/data/mnist.rs:190-199).  No reference output holds concrete weights or a
concrete order, so both are pinned by what mathematics and textbook routines fix:

* the step s ^= s << 13; s ^= s >> 7; s ^= s << 17 is a linear map T over GF(2)^64.  Marsaglia
  ("Xorshift RNGs", J. Stat. Softw. 8(14), 2003) lists (13, 7, 17) among the triples whose T has
  the full period 2^64 - 1; a mistyped shift fails that (checked here as T^(2^64-1) = I and
  T^((2^64-1)/p) != I for every prime p of 2^64 - 1);
* the init seed 0x9E3779B9 is floor(2^32 / phi) (the golden ratio, root of x^2 = x + 1) and the
  shuffle seed 0xD1B54A32D192ED03 is floor(2^64 / phi_3) (phi_3 the real root of x^4 = x + 1,
  the generalised golden ratio of Roberts' R-sequence), both checked in exact rational
  arithmetic;
* the oracle's weights equal the 24-bit grid values of T^i(seed) computed here as repeated
  GF(2) matrix-vector products with the full-period T (swapping the outer shifts, 17/7/13,
  is also full period; this comparison tells the two apart);
* the shuffle equals Python's own ``random.Random.shuffle`` (Durstenfeld's Fisher-Yates from
  the last index down) driven by ``state % n`` draws from T.

Constants that only the reference text fixes (no closed form): the SplitMix64 multiplier
0xBF58476D1CE4E5B9 of the seed fold (nn.rs:662-663)."""

import random
from fractions import Fraction

import numpy as np
import pytest

import oracle

MASK = (1 << 64) - 1
PERIOD = (1 << 64) - 1
PRIMES = (3, 5, 17, 257, 641, 65537, 6700417)


def _step(s: int) -> int:
    s ^= (s << 13) & MASK
    s ^= s >> 7
    s ^= (s << 17) & MASK
    return s


class Gf2:
    """A linear map of GF(2)^64 stored as the images of the 64 basis vectors."""

    def __init__(self, columns):
        self.cols = tuple(columns)

    @staticmethod
    def identity():
        return Gf2(1 << j for j in range(64))

    @staticmethod
    def of(fn):
        return Gf2(fn(1 << j) for j in range(64))

    def apply(self, v: int) -> int:
        out, j = 0, 0
        while v:
            if v & 1:
                out ^= self.cols[j]
            v >>= 1
            j += 1
        return out

    def __matmul__(self, other):  # self after other
        return Gf2(self.apply(c) for c in other.cols)

    def __pow__(self, e: int):
        result, base = Gf2.identity(), self
        while e:
            if e & 1:
                result = base @ result
            base = base @ base
            e >>= 1
        return result

    def __eq__(self, other):
        return self.cols == other.cols


def _shift_map(amount: int, left: bool) -> Gf2:
    return Gf2.of(lambda v: v ^ (((v << amount) & MASK) if left else (v >> amount)))


def test_prime_factorisation_of_the_period():
    prod = 1
    for p in PRIMES:
        assert all(p % d for d in range(2, int(p ** 0.5) + 1))
        prod *= p
    assert prod == PERIOD


def test_xorshift_triple_has_full_period():
    t = _shift_map(17, True) @ _shift_map(7, False) @ _shift_map(13, True)
    assert t == Gf2.of(_step)  # the three shifts compose to one step
    assert t ** PERIOD == Gf2.identity()
    for p in PRIMES:
        assert t ** (PERIOD // p) != Gf2.identity(), p
    # a neighbouring triple is not full period: the check discriminates
    bad = _shift_map(17, True) @ _shift_map(7, False) @ _shift_map(12, True)
    assert bad ** PERIOD != Gf2.identity() or any(
        bad ** (PERIOD // p) == Gf2.identity() for p in PRIMES)


def _floor_inverse_root(bits: int, poly) -> int:
    """floor(2^bits / r) for the root r > 1 of the increasing polynomial ``poly``; verified in
    exact rationals: poly(2^bits / c) >= 0 > poly(2^bits / (c + 1))."""
    lo, hi = Fraction(1), Fraction(2)
    for _ in range(200):  # bisection to far below 2^-bits relative
        mid = (lo + hi) / 2
        lo, hi = (lo, mid) if poly(mid) >= 0 else (mid, hi)
    c = int(Fraction(1 << bits) / hi)
    while poly(Fraction(1 << bits, c + 1)) >= 0:
        c += 1
    while poly(Fraction(1 << bits, c)) < 0:
        c -= 1
    assert poly(Fraction(1 << bits, c)) >= 0 > poly(Fraction(1 << bits, c + 1))
    return c


def test_init_seed_is_the_golden_ratio_constant():
    assert _floor_inverse_root(32, lambda x: x * x - x - 1) == 0x9E3779B9


def test_shuffle_seed_is_the_r3_constant():
    assert _floor_inverse_root(64, lambda x: x ** 4 - x - 1) == 0xD1B54A32D192ED03


def _fold_seed(shape) -> int:
    state = 0x9E3779B9
    for d in shape:
        state ^= (d * 0xBF58476D1CE4E5B9) & MASK
    return state | 1


@pytest.mark.parametrize("shape,ipg", [([4, 2, 3, 3], 2), ([8, 1, 5, 5], 1), ([10, 32, 1, 1], 32)])
def test_init_stream_equals_gf2_matrix_powers(shape, ipg):
    w = oracle.initialized_weights(shape, ipg).ravel()
    t = Gf2.of(_step)
    state, k = _fold_seed(shape), []
    for _ in range(w.size):  # the first value uses the state after one step
        state = t.apply(state)
        k.append(state >> 40)
    kernel_area = shape[2] * shape[3]
    scale = np.sqrt(np.float32(2.0) / np.float32(ipg * kernel_area))
    unit = np.array(k, np.float64).astype(np.float32) / np.float32(1 << 24)
    expect = (unit * np.float32(2.0) - np.float32(1.0)) * scale
    np.testing.assert_array_equal(w, expect.astype(np.float32))


class _XorshiftDraws(random.Random):
    """Python's shuffle with draws ``state % n`` from the xorshift stream."""

    def __init__(self, seed):
        super().__init__(0)
        self.state = seed

    def _randbelow(self, n):
        self.state = _step(self.state)
        return self.state % n


@pytest.mark.parametrize("count", [0, 1, 2, 3, 7, 64, 1000])
def test_shuffle_is_fisher_yates_over_the_stream(count):
    values = list(range(count))
    _XorshiftDraws(0xD1B54A32D192ED03).shuffle(values)
    np.testing.assert_array_equal(oracle.mnist_order(count, True), np.array(values, np.uint64))
