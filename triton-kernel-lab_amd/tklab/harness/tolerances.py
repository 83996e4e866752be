"""Numerical acceptance policies used by the kernel tests.

The per-dtype ``(rtol, atol)`` table and both assertion helpers keep the
reference's thresholds and messages (``src/tklab/harness/tolerances.py:7-85``):
the reference's tests are written against them.
"""

from __future__ import annotations

import torch

# dtype -> (rtol, atol)
_TOLERANCES: dict[torch.dtype, tuple[float, float]] = {
    torch.float16: (1e-2, 1e-2),
    torch.bfloat16: (1.6e-2, 1e-2),
    torch.float32: (1e-4, 1e-5),
}


def dtype_tolerance(dtype: torch.dtype) -> tuple[float, float]:
    """Return the default ``(rtol, atol)`` for ``dtype``.

    Raises:
        ValueError: if no default is configured for ``dtype``.
    """
    try:
        return _TOLERANCES[dtype]
    except KeyError:
        raise ValueError(f"no default tolerance configured for {dtype}") from None


def assert_close(
    output: torch.Tensor,
    reference: torch.Tensor,
    *,
    rtol: float | None = None,
    atol: float | None = None,
) -> None:
    """Elementwise comparison with dtype-aware default tolerances.

    ``reference`` is cast to ``output.dtype`` first, so a float32 reference is
    compared at the precision the kernel stores.

    Raises:
        ValueError: if ``output.dtype`` has no default tolerance.
        AssertionError: if ``output`` holds NaN/Inf or differs beyond tolerance.
    """
    default_rtol, default_atol = dtype_tolerance(output.dtype)
    if not bool(torch.isfinite(output).all()):
        raise AssertionError("output contains non-finite values")
    torch.testing.assert_close(
        output,
        reference.to(output.dtype),
        rtol=default_rtol if rtol is None else rtol,
        atol=default_atol if atol is None else atol,
    )


def relative_frobenius_error(output: torch.Tensor, reference: torch.Tensor) -> float:
    """Return ``||output - reference||_F / ||reference||_F`` in float32.

    When the reference norm is zero the absolute error norm is returned.
    """
    out = output.float()
    ref = reference.float()
    err = torch.linalg.vector_norm(out - ref)
    ref_norm = torch.linalg.vector_norm(ref)
    if ref_norm.item() != 0.0:
        err = err / ref_norm
    return float(err.item())


def assert_relative_frobenius(
    output: torch.Tensor,
    reference: torch.Tensor,
    *,
    max_relative_error: float,
) -> None:
    """Aggregate check for reductions (GEMM, attention, norms).

    Raises:
        ValueError: if ``max_relative_error`` is not positive.
        AssertionError: on non-finite output/reference/error, or an error at or
            above ``max_relative_error``.
    """
    if max_relative_error <= 0:
        raise ValueError("max_relative_error must be positive")
    if not bool(torch.isfinite(output.float()).all()):
        raise AssertionError("output contains non-finite values")
    if not bool(torch.isfinite(reference.float()).all()):
        raise AssertionError("reference contains non-finite values")
    error = relative_frobenius_error(output, reference)
    if error != error or error in (float("inf"), float("-inf")):
        raise AssertionError("relative Frobenius error is non-finite")
    if error >= max_relative_error:
        raise AssertionError(
            f"relative Frobenius error {error:.6g} exceeds {max_relative_error:.6g}"
        )
