"""The LSE comparison of the GPU tests: rows without keys are checked, never skipped (CPU)."""

import numpy as np
import pytest

from tests.gpu_util import lse_max_err

NINF = -np.inf


def test_finite_rows_compared_and_empty_rows_accepted():
    ref = np.array([[1.0, NINF, 3.0]])
    out = np.zeros((1, 3, 2))
    out[0, 0] = 1.0
    out[0, 2] = 2.0
    assert lse_max_err(np.array([[1.25, NINF, 3.0]]), ref, out) == 0.25


@pytest.mark.parametrize("bad", [np.nan, 0.0, 5.0])
def test_empty_row_must_be_neg_inf(bad):
    with pytest.raises(AssertionError):
        lse_max_err(np.array([[1.0, bad]]), np.array([[1.0, NINF]]))


def test_nan_in_a_finite_row_fails():
    with pytest.raises(AssertionError):
        lse_max_err(np.array([[np.nan, 2.0]]), np.array([[1.0, 2.0]]))


def test_empty_row_output_must_be_zero():
    out = np.zeros((1, 2, 4))
    out[0, 1, 3] = 1e-3
    with pytest.raises(AssertionError):
        lse_max_err(np.array([[1.0, NINF]]), np.array([[1.0, NINF]]), out)
