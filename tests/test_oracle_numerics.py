"""Pins the oracle's numeric helpers against torch / exact arithmetic (CPU only)."""
import math
from fractions import Fraction

import numpy as np
import torch

from oracle.numerics import (LN2_F32, bf16_round, bf16_ulp_distance, fma32, ln32,
                             next_pow2)


def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(size=20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
                        np.array([0, -0.0, 1, 1 + 2 ** -8, 1 + 3 * 2 ** -8, np.inf, -np.inf, 3.4e38],
                                 dtype=np.float32)]).astype(np.float32)
    expected = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(bf16_round(x), expected)
    assert np.isnan(bf16_round(np.array([np.nan], dtype=np.float32)))[0]


def test_fma_single_rounding():
    # a*b + c with a product that is not representable in float32.
    a = np.float32(1 + 2 ** -12)
    b = np.float32(1 + 2 ** -12)
    c = np.float32(-(1 + 2 ** -11))
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))   # +2^-24
    assert float(fma32(a, b, c)) == float(exact)
    assert float(np.float32(a * b) + c) == 0.0   # two roundings lose it


def test_ln_by_change_of_base():
    assert LN2_F32 == np.float32(0.6931472)
    xs = np.float32([1e-30, 0.5, 1, 2, 3, 1e10, 123.456])
    np.testing.assert_allclose(ln32(xs), np.log(xs.astype(np.float64)), rtol=3e-7, atol=1e-7)
    assert ln32(np.float32(1)) == 0


def test_ulp_distance():
    one = np.float32(1)
    nxt = np.float32(1 + 2 ** -7)
    assert bf16_ulp_distance(one, nxt) == 1
    assert bf16_ulp_distance(np.float32(0), np.float32(-0.0)) == 0
    assert bf16_ulp_distance(-one, -nxt) == 1
    assert next_pow2(36) == 64 and next_pow2(1) == 1 and next_pow2(64) == 64
    assert math.isclose(float(np.asarray(bf16_round(np.float32(1 / 3))).reshape(-1)[0]), 0.333984375)
