"""CPU tests of the agreement bars in tests/tolerances.py (they back the GPU parity tests and
bench.py's agreement gate)."""
import math

import numpy as np
import pytest

from tests.tolerances import assert_grads_close, grad_error


def _pair(n=100_000, seed=0):
    rng = np.random.default_rng(seed)
    want = rng.standard_normal(n).astype(np.float32)
    return want.copy(), want


def test_identical_gradients_pass():
    got, want = _pair()
    assert grad_error(got, want) == (0.0, 0.0)
    assert_grads_close(["g"], [got], [want])


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_one_non_finite_value_fails(bad):
    got, want = _pair()
    got[12345] = bad
    outside, rel = grad_error(got, want)
    assert math.isinf(rel) and outside > 0
    with pytest.raises(AssertionError):
        assert_grads_close(["g"], [got], [want])


def test_non_finite_values_fail_in_every_chunk():
    got, want = _pair(n=10_000)
    got[[3, 5003, 9999]] = np.nan
    outside, rel = grad_error(got, want, chunk=1000)
    assert math.isinf(rel) and outside == pytest.approx(3 / 10_000)


def test_a_few_values_outside_pass_and_a_large_error_fails():
    got, want = _pair()
    got[:50] += 0.01 * np.abs(want).max()          # 0.05% outside rtol, max error 1e-2 of max|want|
    with pytest.raises(AssertionError, match="max error"):
        assert_grads_close(["g"], [got], [want])
    got, want = _pair()
    got[:50] += 1e-3 * np.abs(want).max()          # 0.05% outside, max error 1e-3: within both bars
    assert_grads_close(["g"], [got], [want])
    got[:200] += 1e-3 * np.abs(want).max()         # 0.2% outside: fails the share bar
    with pytest.raises(AssertionError, match="outside tolerance"):
        assert_grads_close(["g"], [got], [want])
