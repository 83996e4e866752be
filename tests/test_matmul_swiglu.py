"""GPU parity of tk_gemm_swiglu: bitwise against the unfused GEMM + SwiGLU kernels,
and against the CPU oracle (GEMM then SwiGLU) within the dtype tolerance."""

from __future__ import annotations

import pytest
import torch

from _helpers import bits_equal, dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close
from tklab.kernels.matmul import matmul_fp32acc
from tklab.kernels.matmul_swiglu import fused_applies, matmul_swiglu
from tklab.kernels.swiglu import swiglu

pytestmark = pytest.mark.gpu


def _operands(m, n, k, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    sc = k ** -0.25
    x = (torch.randn(m, k, device="cuda", generator=g) * sc).to(dtype)
    wg = (torch.randn(k, n, device="cuda", generator=g) * sc).to(dtype)
    wu = (torch.randn(k, n, device="cuda", generator=g) * sc).to(dtype)
    return x, wg, wu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "m,n,k", [(1, 8, 32), (8, 8, 32), (256, 128, 64), (300, 520, 96), (257, 136, 160),
              (1000, 1032, 256), (2048, 1024, 512), (300, 264, 1056)]
)
def test_fused_is_bitwise_the_unfused_composition(dtype, m, n, k) -> None:
    x, wg, wu = _operands(m, n, k, dtype, seed=m + n + k)
    assert fused_applies(x, wg, wu)
    y = matmul_swiglu(x, wg, wu)
    ref = swiglu(matmul_fp32acc(x, wu), matmul_fp32acc(x, wg))
    assert bits_equal(y, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_matches_the_oracle(dtype) -> None:
    x, wg, wu = _operands(200, 264, 128, dtype, seed=11)
    y = matmul_swiglu(x, wg, wu)
    gate = oracle.gemm(host(x), host(wg), name(dtype))
    value = oracle.gemm(host(x), host(wu), name(dtype))
    assert_close(y, dev(oracle.swiglu_fwd(value, gate, name(dtype)), y))


def test_strided_and_ragged_problems_take_the_composition() -> None:
    x, wg, wu = _operands(100, 72, 40, torch.bfloat16, seed=12)  # k % 32 != 0
    assert not fused_applies(x, wg, wu)
    assert bits_equal(matmul_swiglu(x, wg, wu), swiglu(matmul_fp32acc(x, wu), matmul_fp32acc(x, wg)))
    xs = torch.randn(64, 2 * 96, device="cuda", dtype=torch.bfloat16)[:, ::2]  # column stride 2
    _, wg2, wu2 = _operands(64, 64, 96, torch.bfloat16, seed=13)
    assert not fused_applies(xs, wg2, wu2)
    assert bits_equal(matmul_swiglu(xs, wg2, wu2),
                      swiglu(matmul_fp32acc(xs, wu2), matmul_fp32acc(xs, wg2)))


def test_weight_row_strides_may_differ() -> None:
    x, wg, _ = _operands(128, 256, 64, torch.bfloat16, seed=14)
    wu_storage = torch.randn(64, 384, device="cuda", dtype=torch.bfloat16)
    wu = wu_storage[:, 64:320]
    assert fused_applies(x, wg, wu)
    assert bits_equal(matmul_swiglu(x, wg, wu), swiglu(matmul_fp32acc(x, wu), matmul_fp32acc(x, wg)))


def test_extreme_gates_stay_finite() -> None:
    x = torch.eye(64, device="cuda", dtype=torch.bfloat16)
    wg = torch.full((64, 64), 90.0, device="cuda", dtype=torch.bfloat16)
    wg[:, 32:] = -90.0
    wu = torch.ones(64, 64, device="cuda", dtype=torch.bfloat16)
    y = matmul_swiglu(x, wg, wu)
    assert torch.isfinite(y.float()).all()
    assert torch.all(y[:, :32] == 90.0) and torch.all(y[:, 32:] <= 0)
