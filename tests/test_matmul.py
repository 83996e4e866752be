"""GPU parity of tk_gemm (matmul_fp32acc / matmul_fp16acc).

Reference checks: relative Frobenius < 1e-2 against torch.matmul on float32
upcasts (reference matmul.py:282-284) on square, tail and strided problems.
This build adds the CPU oracle (double accumulation) on sampled rows at the
benchmark shapes and elementwise agreement at the storage dtype's tolerance.
"""

from __future__ import annotations

import pytest
import torch

from _helpers import dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.matmul import _make_adversarial, matmul_fp16acc, matmul_fp32acc

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _inputs(m: int, n: int, k: int, dtype: torch.dtype):
    # N(0, 1/sqrt(K)) entries: randn * K^(-1/4), so C has unit variance.
    scale = k ** -0.25
    a = (torch.randn(m, k, device="cuda") * scale).to(dtype)
    b = (torch.randn(k, n, device="cuda") * scale).to(dtype)
    return a, b


def _check_rows(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, rows: torch.Tensor) -> None:
    expected = oracle.gemm(host(a[rows]), host(b), name(a.dtype))
    got = c[rows]
    assert_close(got, dev(expected, got))
    assert_relative_frobenius(got, dev(expected, got), max_relative_error=1e-3)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(
    ("m", "n", "k"),
    [(1, 1, 8), (1, 8, 1), (8, 8, 8), (256, 256, 64), (300, 520, 72), (512, 512, 512),
     (129, 257, 193), (1024, 1024, 1024), (255, 264, 4096), (7, 9, 11),
     # K % 32 == 0 goes through the DMA kernel: fewer K tiles than the prefetch depth,
     # exactly the prefetch depth, and M/N edges inside one block tile; K = 1056 is an
     # odd count of 32-wide steps (last 64-wide A tile half used) after many ring wraps.
     (1, 8, 32), (33, 40, 32), (300, 520, 96), (257, 136, 160), (520, 1032, 128),
     (520, 264, 1056)],
)
def test_small_shapes_match_the_oracle(dtype: torch.dtype, m: int, n: int, k: int) -> None:
    torch.manual_seed(m * 7 + n * 3 + k)
    a, b = _inputs(m, n, k, dtype)
    c = matmul_fp32acc(a, b)
    _check_rows(a, b, c, torch.arange(m, device="cuda"))
    assert_relative_frobenius(c, a.float() @ b.float(), max_relative_error=1e-2)


def test_strided_adversarial_tails() -> None:
    torch.manual_seed(0)
    a, b = _make_adversarial(torch.device("cuda"))
    assert a.stride(1) == 2 and b.stride(0) == 2 * 257
    c = matmul_fp32acc(a, b)
    _check_rows(a, b, c, torch.arange(a.shape[0], device="cuda"))
    assert_relative_frobenius(c, a.float() @ b.float(), max_relative_error=1e-2)
    assert_relative_frobenius(matmul_fp16acc(a, b), a.float() @ b.float(), max_relative_error=5e-2)


def test_transposed_views_take_the_general_path() -> None:
    torch.manual_seed(1)
    a = torch.randn(96, 80, device="cuda", dtype=torch.float16).t()  # (80, 96), column-major
    b = torch.randn(72, 96, device="cuda", dtype=torch.float16).t()  # (96, 72)
    c = matmul_fp32acc(a, b)
    _check_rows(a, b, c, torch.arange(80, device="cuda"))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("m", "n", "k"), [(4096, 4096, 4096), (8191, 8192, 8192), (8192, 8192, 8192)])
def test_config_shapes(dtype: torch.dtype, m: int, n: int, k: int) -> None:
    """benchmark config 4: 8192^3 (and 4096^3, ragged M=8191), N(0, 1/sqrt(K)) inputs."""
    torch.manual_seed(0)
    a, b = _inputs(m, n, k, dtype)
    c = matmul_fp32acc(a, b)
    assert torch.isfinite(c).all()
    rows = torch.cat([torch.arange(0, m, 997, device="cuda"), torch.tensor([m - 1], device="cuda")])
    _check_rows(a, b, c, rows)
    # The whole of C, elementwise, against float32 math on the same operands (the
    # reference's matmul.py:282-284 compares the float32 product; tolerances.py:7-11 gives
    # the storage dtype's atol/rtol), so an error confined to a few tiles cannot pass.
    want = a.float() @ b.float()
    assert_close(c, want)
    assert_relative_frobenius(c, want, max_relative_error=1e-2)


def test_linearity_in_the_left_operand() -> None:
    torch.manual_seed(2)
    a1, b = _inputs(512, 384, 640, torch.float16)
    a2, _ = _inputs(512, 384, 640, torch.float16)
    lhs = matmul_fp32acc((a1.float() + a2.float()).half(), b).float()
    rhs = matmul_fp32acc(a1, b).float() + matmul_fp32acc(a2, b).float()
    assert_relative_frobenius(lhs, rhs, max_relative_error=5e-3)


def test_identity_is_exact() -> None:
    torch.manual_seed(3)
    a = torch.randn(384, 264, device="cuda", dtype=torch.bfloat16)
    eye = torch.eye(264, device="cuda", dtype=torch.bfloat16)
    assert torch.equal(matmul_fp32acc(a, eye), a)


@pytest.mark.parametrize("k", [264, 256])
def test_identity_is_exact_on_both_paths(k: int) -> None:
    """K = 264 takes the register-staged kernel, K = 256 the DMA kernel."""
    torch.manual_seed(4)
    a = torch.randn(300, k, device="cuda", dtype=torch.float16)
    eye = torch.eye(k, device="cuda", dtype=torch.float16)
    assert torch.equal(matmul_fp32acc(a, eye), a)
