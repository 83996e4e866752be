"""Tolerance helpers (same cases as the reference's tests/test_tolerances.py)."""

from __future__ import annotations

import pytest
import torch

from tklab.harness.tolerances import (
    assert_close,
    assert_relative_frobenius,
    dtype_tolerance,
    relative_frobenius_error,
)


def test_default_table_matches_the_reference_policy() -> None:
    assert dtype_tolerance(torch.float16) == (1e-2, 1e-2)
    assert dtype_tolerance(torch.bfloat16) == (1.6e-2, 1e-2)
    assert dtype_tolerance(torch.float32) == (1e-4, 1e-5)
    with pytest.raises(ValueError, match="no default tolerance"):
        dtype_tolerance(torch.int32)


def test_half_precision_rounding_error_is_accepted() -> None:
    assert_close(torch.tensor([1.0, 2.0], dtype=torch.float16), torch.tensor([1.001, 2.001]))


def test_nan_output_fails_even_with_huge_tolerances() -> None:
    out = torch.tensor([float("nan")])
    with pytest.raises(AssertionError, match="non-finite"):
        assert_close(out, torch.zeros(1), rtol=1.0, atol=1.0)


def test_zero_reference_uses_the_absolute_norm() -> None:
    assert relative_frobenius_error(torch.zeros(4), torch.zeros(4)) == 0.0
    assert_relative_frobenius(torch.zeros(4), torch.zeros(4), max_relative_error=1e-3)
    assert relative_frobenius_error(torch.full((4,), 0.5), torch.zeros(4)) == pytest.approx(1.0)


def test_large_aggregate_error_fails() -> None:
    with pytest.raises(AssertionError, match="Frobenius"):
        assert_relative_frobenius(torch.ones(4), torch.zeros(4), max_relative_error=0.5)


def test_threshold_is_strict() -> None:
    out = torch.tensor([1.1, 0.0])
    ref = torch.tensor([1.0, 0.0])
    with pytest.raises(AssertionError):
        assert_relative_frobenius(out, ref, max_relative_error=0.1 - 1e-7)
    assert_relative_frobenius(out, ref, max_relative_error=0.11)


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), -float("inf")])
def test_non_finite_reference_fails(bad: float) -> None:
    ref = torch.tensor([bad])
    with pytest.raises(AssertionError, match="reference contains non-finite"):
        assert_relative_frobenius(torch.zeros(1), ref, max_relative_error=1e-3)


def test_non_positive_threshold_is_a_usage_error() -> None:
    with pytest.raises(ValueError, match="positive"):
        assert_relative_frobenius(torch.zeros(1), torch.zeros(1), max_relative_error=0.0)
