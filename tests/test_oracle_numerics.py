"""Pins the canonical primitives of the oracle against libm in double
precision: the canonical exp/log1p must stay within a few ulp of the true
value, bf16 rounding must be round-to-nearest-even, and the L64 reduction
must equal an exact (fp64) sum to fp32 accuracy."""
import math

import numpy as np
import pytest

from _hai import orc


def ulp_err(got, exact):
    got = np.asarray(got, np.float64)
    exact = np.asarray(exact, np.float64)
    sp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    return np.abs(got - exact) / sp


def test_exp_within_2_ulp():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-87, 88.5, 400000), rng.uniform(-2, 2, 200000),
                        np.linspace(-87.3, 88.7, 100001)]).astype(np.float32)
    got = orc.cexp(x)
    exact = np.exp(x.astype(np.float64))
    assert ulp_err(got, exact).max() <= 2.0


def test_exp_special_values():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 89.0, -104.5, -100.0, 1e-30], np.float32)
    y = orc.cexp(x)
    assert y[0] == 1.0 and y[1] == 1.0 and y[2] == np.inf and y[3] == 0.0 and np.isnan(y[4])
    assert y[5] == np.inf and y[6] == 0.0
    assert 0 < y[7] < 1e-43  # subnormal result
    assert abs(y[7] - math.exp(-100.0)) <= np.spacing(np.float32(0)) * 1.0
    assert y[8] == 1.0


def test_log1p_within_3_ulp():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-0.999, 1.0, 300000), rng.uniform(0, 1e-3, 100000),
                        rng.uniform(1, 1e6, 100000), 10.0 ** rng.uniform(-30, -3, 100000)]).astype(np.float32)
    got = orc.clog1p(x)
    exact = np.log1p(x.astype(np.float64))
    assert ulp_err(got, exact).max() <= 3.0


def test_softplus_path_accuracy():
    # the DeltaNet decay uses log1p(exp(-|x|)) for |x| in the range of dt_bias + a
    x = np.linspace(-30, 30, 200001).astype(np.float32)
    got = orc.clog1p(orc.cexp(-np.abs(x)))
    exact = np.log1p(np.exp(-np.abs(x).astype(np.float64)))
    assert ulp_err(got, exact).max() <= 4.0


def test_bf16_round_nearest_even():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(100000).astype(np.float32) * 10
    r = orc.round_bf16(x).astype(np.float64)
    # nearest: error at most half a bf16 ulp
    half = np.spacing(np.abs(r).astype(np.float32)).astype(np.float64) * 2 ** 16 / 2
    assert np.all(np.abs(r - x) <= half * (1 + 1e-12))
    # ties go to the even mantissa
    ties = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, 256 + 1], np.float32)
    assert list(orc.round_bf16(ties)) == [1.0, 1 + 2 ** -6, 256.0]


def test_l64_reduction_accuracy_and_order_dependence():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, 5120)) * 0.3).astype(np.float32)
    w = (rng.standard_normal((7, 5120)) * 0.02).astype(np.float32)
    got = orc.gemm(x, w, round_out=False)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(got, exact, rtol=1e-5, atol=1e-6)
    # row independence: a row's bits do not depend on the other rows
    single = orc.gemm(x[1:2], w, round_out=False)
    assert np.array_equal(single[0], got[1])


def test_l64_gemm_bruteforce_small():
    rng = np.random.default_rng(4)
    for K in (8, 24, 512, 1000):
        x = orc.round_bf16(rng.standard_normal((2, K)).astype(np.float32))
        w = orc.round_bf16(rng.standard_normal((5, K)).astype(np.float32))
        got = orc.gemm(x, w, round_out=False)
        exact = x.astype(np.float64) @ w.astype(np.float64).T
        bound = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T * K * 2 ** -24
        assert np.all(np.abs(got - exact) <= bound + 1e-30)
