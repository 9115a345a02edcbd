"""The tests' numpy restatement of the int8-plane split (tests/planes_np.py), pinned by what the split must meet
whatever its arithmetic, so that the GPU test's bit-for-bit comparison with it checks the kernel against the
property rather than against a copy of the kernel's formula."""
import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from tests.planes_np import split_i8_np

BOUND = 0.5 / 254 ** 2 + 2.0 ** -24   # of S: what three planes of ratio 254 leave


def held(a0, a1, a2, S):
    return S.astype(np.float64)[:, None] * (a0 + (a1.astype(np.float64) + a2 / 254) / 254)


@settings(max_examples=60, deadline=None)
@given(st.integers(0, 2 ** 32 - 1), st.integers(-100, 100), st.integers(1, 6))
def test_split_meets_its_bounds(seed, scale_exp, rows):
    rng = np.random.default_rng(seed)
    v = (rng.standard_normal((rows, 256)) * np.exp2(scale_exp + rng.integers(-8, 8, (rows, 1)))).astype(np.float32)
    v[rng.random(v.shape) < 0.05] = 0.0
    v[0, rng.integers(0, 256)] *= 1000   # an outlier: the other values sit far below the row's largest
    a0, a1, a2, S = split_i8_np(v)
    for a in (a0, a1, a2):
        assert np.all(np.abs(a) <= 127) and np.all(a == np.rint(a))
    m = np.abs(v).max(axis=1).astype(np.float64)
    assert np.all(np.exp2(np.round(np.log2(S))) == S)
    assert np.all(m <= 127 * S.astype(np.float64)) and np.all(m > 63.5 * S.astype(np.float64))
    err = np.abs(held(a0, a1, a2, S) - v)
    assert np.all(err <= BOUND * S.astype(np.float64)[:, None])
    assert np.all(err <= 1.25e-7 * m[:, None])


def test_bound_has_teeth():
    """Two planes leave far more than the bound: the check above would catch a dropped third plane."""
    v = np.random.default_rng(1).standard_normal((8, 256)).astype(np.float32)
    a0, a1, a2, S = split_i8_np(v)
    err = np.abs(held(a0, a1, np.zeros_like(a2), S) - v)
    assert err.max() > 100 * BOUND * S.max()


def test_special_rows():
    v = np.zeros((4, 256), np.float32)
    v[0] = (np.arange(256) % 255 - 127) * 0.25   # integers times a power of two: a0 alone, exactly
    v[1, 3] = np.inf
    v[2, 9] = np.nan
    a0, a1, a2, S = split_i8_np(v)
    assert S[0] == 0.25 and np.array_equal(a0[0] * S[0], v[0]) and not a1[0].any() and not a2[0].any()
    assert np.isnan(S[1]) and np.isnan(S[2]) and S[3] == 0.0
    for r in (1, 2, 3):
        assert not (a0[r].any() or a1[r].any() or a2[r].any())


@pytest.mark.parametrize("m", [2.0 ** -140, 1e-30, 1.0, 127.0, 127.5, 3e38])
def test_scale_is_the_smallest_power_of_two(m):
    v = np.full((1, 256), m / 3, np.float32)
    v[0, 0] = m
    S = split_i8_np(v)[3][0]
    mm = np.float64(np.float32(m))
    assert mm <= 127 * np.float64(S) and (mm > 63.5 * np.float64(S) or S == 2.0 ** -149)
