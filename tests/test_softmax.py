"""GPU parity of tk_softmax_fwd against the CPU oracle and torch.softmax."""

from __future__ import annotations

import pytest
import torch

from _helpers import dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.fused_softmax import _launch, softmax

pytestmark = pytest.mark.gpu


def _check(x: torch.Tensor) -> None:
    y = softmax(x)
    expected = dev(oracle.softmax(host(x), name(x.dtype)), y)
    # Tolerances of the dtype table (float32: rtol 1e-4, atol 1e-5).
    assert_close(y, expected)
    assert_close(y, torch.softmax(x.float(), dim=-1))


def test_config_shape_float32_4096x4096() -> None:
    torch.manual_seed(0)
    x = torch.randn(4096, 4096, device="cuda")
    y = softmax(x)
    expected = dev(oracle.softmax(host(x), "float32"), y)
    assert_close(y, expected)
    assert_relative_frobenius(y, expected, max_relative_error=1e-5)
    rows = y.double().sum(dim=1)
    torch.testing.assert_close(rows, torch.ones_like(rows), rtol=0, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [1, 3, 64, 128, 1000, 1024, 4096, 4097, 8192, 16384, 65536])
def test_widths_and_dtypes(dtype: torch.dtype, cols: int) -> None:
    torch.manual_seed(cols)
    _check(torch.randn(37, cols, device="cuda", dtype=dtype))


def test_row_strided_adversarial_view() -> None:
    torch.manual_seed(0)
    x = torch.randn(64, 1000, device="cuda")[::2]
    _check(x)


def test_misaligned_base_uses_the_scalar_path() -> None:
    torch.manual_seed(1)
    storage = torch.randn(33 * 512 + 1, device="cuda")
    x = storage[1:].view(33, 512)
    _check(x)


def test_launch_writes_into_a_strided_output() -> None:
    torch.manual_seed(2)
    x = torch.randn(16, 256, device="cuda")
    out_storage = torch.full((16, 512), 7.0, device="cuda")
    out = out_storage[:, :256]
    _launch((x,), out)
    assert_close(out, torch.softmax(x, dim=-1))
    assert torch.all(out_storage[:, 256:] == 7.0)


def test_constant_rows_are_uniform_and_large_values_stay_finite() -> None:
    x = torch.full((4, 1000), 3.0, device="cuda")
    x[1] = 1e30
    x[2, :500] = -1e30
    y = softmax(x)
    assert torch.isfinite(y).all()
    torch.testing.assert_close(y[0], torch.full_like(y[0], 1e-3), rtol=1e-6, atol=0)
    torch.testing.assert_close(y[2, 500:], torch.full_like(y[2, 500:], 2e-3), rtol=1e-6, atol=0)
    assert torch.all(y[2, :500] == 0)
