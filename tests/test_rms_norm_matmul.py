"""GPU parity of the normalized GEMM (tk_rmsnorm_fwd statistics mode, tk_scale_rows,
tk_gemm_rowscale) behind residual_rms_norm_matmul.

Each piece is pinned exactly, and the whole against float64:
- the statistics mode writes the same s and rstd bits as the full forward;
- the fold is torch's float32 product w[k] * W[k, n] rounded to the dtype;
- the row-scaled epilogue with unit scales is the plain GEMM bit for bit, and with
  power-of-two scales is the plain GEMM times those scales bit for bit (scaling by
  2^e commutes with rounding away from overflow and subnormals);
- the fused result is no further from the float64 product of the same inputs than
  the composition residual_rms_norm -> matmul_fp32acc is.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits_equal
from tklab import _hip
from tklab.kernels.matmul import matmul_fp32acc
from tklab.kernels.residual_rms_norm import residual_rms_norm
from tklab.kernels.rms_norm_matmul import (
    fold_norm_weight,
    residual_rms_norm_matmul,
    rms_norm_matmul,
)

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]


def _inputs(m, k, n, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", dtype=dtype, generator=g)
    r = torch.randn(m, k, device="cuda", dtype=dtype, generator=g)
    w = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(dtype)
    proj = (torch.randn(k, n, device="cuda", generator=g) * k ** -0.5).to(dtype)
    return x, r, w, proj


def _rowscale(a, b, scale):
    out = torch.empty(a.shape[0], b.shape[1], device="cuda", dtype=a.dtype)
    _hip.call("tk_gemm_rowscale", _hip.dtype_code(a.dtype), a.data_ptr(), b.data_ptr(),
              scale.data_ptr(), out.data_ptr(), a.shape[0], b.shape[1], a.shape[1],
              a.stride(0), a.stride(1), b.stride(0), b.stride(1), out.stride(0), out.stride(1),
              _hip.stream_of(a))
    return out


@pytest.mark.parametrize("dtype", DTYPES)
def test_statistics_mode_writes_the_full_forwards_s_and_rstd(dtype) -> None:
    x, r, w, _ = _inputs(777, 4096, 8, dtype, seed=1)
    rows, cols = x.shape
    full = [torch.empty_like(x), torch.empty_like(x), torch.empty(rows, device="cuda")]
    stats = [torch.empty_like(x), torch.empty(rows, device="cuda")]
    for s, y, rstd in ((full[0], full[1], full[2]), (stats[0], None, stats[1])):
        _hip.call("tk_rmsnorm_fwd", _hip.dtype_code(dtype), x.data_ptr(), r.data_ptr(),
                  w.data_ptr(), s.data_ptr(), None if y is None else y.data_ptr(),
                  rstd.data_ptr(), rows, cols, cols, cols, cols, cols, 1e-6, _hip.stream_of(x))
    assert bits_equal(stats[0], full[0])
    assert bits_equal(stats[1], full[2])


@pytest.mark.parametrize("dtype", DTYPES)
def test_fold_is_the_rounded_float32_product(dtype) -> None:
    _, _, w, proj = _inputs(8, 1000, 328, dtype, seed=2)
    want = (w.float()[:, None] * proj.float()).to(dtype)
    assert bits_equal(fold_norm_weight(w, proj), want)
    # Row-sliced projection (row stride > columns).
    wide = torch.randn(1000, 512, device="cuda").to(dtype)
    got = fold_norm_weight(w, wide[:, :328])
    assert bits_equal(got, (w.float()[:, None] * wide[:, :328].float()).to(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,k", [(256, 512), (1000, 512), (300, 96)])
def test_unit_and_power_of_two_row_scales_are_exact(dtype, m, k) -> None:
    """k = 96: an odd count of 32-wide K steps, so the last 64-wide A tile is half used."""
    x, _, _, proj = _inputs(m, k, 264, dtype, seed=3 + m)
    plain = matmul_fp32acc(x, proj)
    ones = torch.ones(m, device="cuda")
    assert bits_equal(_rowscale(x, proj, ones), plain)
    e = torch.randint(-3, 4, (m,), device="cuda", generator=torch.Generator(device="cuda").manual_seed(m))
    scale = torch.pow(2.0, e.float())
    want = (plain.float() * scale[:, None]).to(dtype)
    got = _rowscale(x, proj, scale)
    # float16 values scaled across its subnormal range (below 2^-14) lose bits either
    # way; compare where the plain value stays normal after a 2^-3 scale.
    normal = plain.float().abs() >= 2.0 ** -11
    assert normal.float().mean().item() > 0.99
    assert bits_equal(got[normal], want[normal])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,k,n", [(512, 1024, 768), (300, 4096, 1032)])
def test_no_less_accurate_than_the_composition(dtype, m, k, n) -> None:
    x, r, w, proj = _inputs(m, k, n, dtype, seed=m + n)
    s, out = residual_rms_norm_matmul(x, r, fold_norm_weight(w, proj), eps=1e-6)
    s_ref, y_ref = residual_rms_norm(x, r, w, eps=1e-6)
    assert bits_equal(s, s_ref)
    composed = matmul_fp32acc(y_ref, proj)
    # float64 product of the same storage-precision inputs.
    s64 = s.double().cpu().numpy()
    rstd = 1.0 / np.sqrt((s64 * s64).mean(axis=1, keepdims=True) + 1e-6)
    exact = (s64 * rstd * w.double().cpu().numpy()) @ proj.double().cpu().numpy()
    err_fused = np.linalg.norm(out.double().cpu().numpy() - exact)
    err_comp = np.linalg.norm(composed.double().cpu().numpy() - exact)
    assert err_fused / np.linalg.norm(exact) < 1e-2
    assert err_fused <= 1.25 * err_comp, (err_fused, err_comp)


def test_without_residual_equals_the_residual_form_on_zero_residual() -> None:
    x, _, w, proj = _inputs(384, 2048, 512, torch.bfloat16, seed=9)
    folded = fold_norm_weight(w, proj)
    s, with_zero = residual_rms_norm_matmul(x, torch.zeros_like(x), folded)
    assert bits_equal(s, x)
    assert bits_equal(rms_norm_matmul(x, folded), with_zero)


def test_contract() -> None:
    x, r, w, proj = _inputs(64, 512, 64, torch.bfloat16, seed=10)
    folded = fold_norm_weight(w, proj)
    with pytest.raises(ValueError, match="residual must match"):
        residual_rms_norm_matmul(x, r[:, :256], folded)
    with pytest.raises(ValueError, match="incompatible shapes"):
        rms_norm_matmul(x, folded[:256])
    with pytest.raises(ValueError, match="finite and positive"):
        rms_norm_matmul(x, folded, eps=0.0)
    with pytest.raises(ValueError, match="K % 32 == 0"):
        rms_norm_matmul(x[:, :500], fold_norm_weight(w[:500], proj[:500]))
    with pytest.raises(ValueError, match="input dimension"):
        fold_norm_weight(w[:10], proj)
