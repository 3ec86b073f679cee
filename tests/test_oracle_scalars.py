"""Pins the oracle's scalar building blocks (oracle/q27o.c) against independent references:
bf16 round-to-nearest-even (include/q27.h:136-139) against a float64 nearest-neighbour search,
and the portable exp / exp2 / log1p / sigmoid / SiLU / softplus (src/q27_gdn.hip:114-119, 317)
against numpy's float64 libm within stated ulp bounds."""
import numpy as np
import pytest

import ref64


def vec(O, x, op):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    O.lib().q27o_math_vec(x.ctypes.data, y.ctypes.data, x.size, op)
    return y


def ulp_err(got, ref):
    got = got.astype(np.float64)
    ref = np.asarray(ref, np.float64)
    sp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return np.abs(got - ref) / sp


def test_bf16_rne_matches_nearest_search(O):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 200000),
        # exact ties: low 16 bits 0x8000, both parities of the kept LSB
        (rng.integers(0x00800000, 0x7F000000, 4000, dtype=np.uint32) & 0xFFFF0000 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.005859375, 3e38, -3e38, 1e-40], np.float32),
    ]).astype(np.float32)
    got = np.array([O.lib().q27o_f2bf(float(v)) for v in x[:3000]], np.uint16)
    assert np.array_equal(got, ref64.bf16_rne(x[:3000]))
    assert np.array_equal(O.f2bf(x), ref64.bf16_rne(x))   # vectorized twin used by the tests
    # known answers: 1 + 2^-8 is a tie between 1 and 1 + 2^-7 -> even (1.0); 1 + 3*2^-8 -> up
    assert O.lib().q27o_f2bf(1.00390625) == 0x3F80
    assert O.lib().q27o_f2bf(1.01171875) == 0x3F82
    assert O.lib().q27o_bf2f(0x3F80) == 1.0 and O.lib().q27o_bf2f(0xC000) == -2.0


def test_exp_accuracy(O):
    x = np.concatenate([np.linspace(-87.3, 88.7, 400001, dtype=np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 0.5, -0.5], np.float32)])
    y = vec(O, x, 0)
    assert ulp_err(y, np.exp(x.astype(np.float64))).max() <= 2.0
    assert vec(O, np.array([0.0], np.float32), 0)[0] == 1.0
    assert vec(O, np.array([89.0, -104.0, np.inf, -np.inf], np.float32), 0).tolist() == [np.inf, 0.0, np.inf, 0.0]
    # subnormal results: absolute error below one subnormal step
    xs = np.linspace(-103.0, -87.4, 20001, dtype=np.float32)
    assert np.abs(vec(O, xs, 0).astype(np.float64) - np.exp(xs.astype(np.float64))).max() <= 2 * 1.4e-45


def test_exp2_accuracy(O):
    x = np.linspace(-126.0, 127.9, 400001, dtype=np.float32)
    assert ulp_err(vec(O, x, 1), np.exp2(x.astype(np.float64))).max() <= 2.0
    ints = np.arange(-126, 128, dtype=np.float32)
    assert np.array_equal(vec(O, ints, 1), np.exp2(ints.astype(np.float64)).astype(np.float32))  # exact powers of two


def test_log1p_accuracy(O):
    x = np.concatenate([np.linspace(-0.999, 10.0, 200001, dtype=np.float32),
                        np.logspace(-12, 30, 20001).astype(np.float32),
                        -np.logspace(-12, -0.0005, 20001).astype(np.float32)])
    assert ulp_err(vec(O, x, 2), np.log1p(x.astype(np.float64))).max() <= 4.0
    tiny = np.array([1e-30, -1e-30, 1e-9], np.float32)
    assert np.array_equal(vec(O, tiny, 2), tiny)                     # log1p(y) = y below the 1+y rounding


@pytest.mark.parametrize("op,fn,lo,hi", [(3, ref64.sigmoid, -80, 80), (4, ref64.silu, -80, 80),
                                          (5, ref64.softplus, -80, 80)])
def test_activations(O, op, fn, lo, hi):
    x = np.linspace(lo, hi, 200001, dtype=np.float32)
    y = vec(O, x, op)
    ref = fn(x.astype(np.float64))
    # sigmoid / SiLU / softplus are one or two roundings past exp: relative 1e-6, absolute near 0
    assert (np.abs(y - ref) <= 1e-6 * np.abs(ref) + 1e-30).all()


def test_softplus_passthrough(O):
    """softplus(x) = x exactly for x > 20 (src/q27_gdn.hip:317)."""
    x = np.array([20.000002, 25.0, 88.0, 1e6], np.float32)
    assert np.array_equal(vec(O, x, 5), x)


def test_generator_moments(O):
    """The shared synthetic generator: N(0,1) draws have mean 0 / variance 1 / bounded support,
    uniform draws lie in [0,1) with mean 1/2; and both are pure functions of (seed, tensor, idx)."""
    L = O.lib()
    n = np.array([L.q27o_normal(7, 3, i) for i in range(40000)])
    assert abs(n.mean()) < 0.03 and abs(n.var() - 1) < 0.03 and np.abs(n).max() < 3.47
    u = np.array([L.q27o_uniform(7, 4, i) for i in range(40000)])
    assert u.min() >= 0 and u.max() < 1 and abs(u.mean() - 0.5) < 0.01
    assert L.q27o_normal(7, 3, 5) == L.q27o_normal(7, 3, 5)
    assert L.q27o_hash(7, 3, 5) != L.q27o_hash(7, 3, 6) != L.q27o_hash(8, 3, 5)
