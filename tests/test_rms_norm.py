"""GPU parity of the RMSNorm kernels (forward, stage 1, stage 2, autograd).

Reference cases (seeds 0-3, shapes, thresholds) follow the reference's
tests/test_rms_norm.py; the oracle comparisons and the determinism checks are
this build's own.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from _helpers import bits_equal, dev, host, name, strided_rows
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels import _norm_common
from tklab.kernels.rms_norm import (
    _launch_backward_stage1,
    _launch_backward_stage2,
    _launch_forward,
    _make_backward_buffers,
    rms_norm,
)

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _problem(rows: int = 37, cols: int = 1000):
    x = strided_rows(rows, cols, 2, requires_grad=True)
    dy = strided_rows(rows, cols, 3)
    w = torch.randn(cols, device="cuda", requires_grad=True)
    return x, w, dy


def test_forward_matches_pytorch_on_strided_tail() -> None:
    torch.manual_seed(0)
    x, w, _ = _problem()
    y = rms_norm(x, w)
    assert_relative_frobenius(y, F.rms_norm(x, (x.shape[-1],), w, EPS), max_relative_error=1e-4)


@pytest.mark.parametrize("rows", [67, 1025])
def test_gradients_match_autograd(rows: int) -> None:
    torch.manual_seed(1 if rows == 67 else 2)
    x, w, dy = _problem(rows=rows)
    ref = F.rms_norm(x, (x.shape[-1],), w, EPS)
    dx_ref, dw_ref = torch.autograd.grad(ref, (x, w), grad_outputs=dy)
    x2 = x.detach().requires_grad_(True)
    w2 = w.detach().requires_grad_(True)
    dx, dw = torch.autograd.grad(rms_norm(x2, w2), (x2, w2), grad_outputs=dy)
    assert_relative_frobenius(dx, dx_ref, max_relative_error=1e-2)
    assert_relative_frobenius(dw, dw_ref, max_relative_error=1e-2)


def test_single_group_state_and_gradient_over_repeated_runs() -> None:
    torch.manual_seed(3)
    rows, cols = 1025, 1000
    x, w, dy = _problem(rows=rows, cols=cols)
    out = torch.empty_like(x)
    rstd = torch.empty(rows, device="cuda")
    _launch_forward(x, w, out, rstd, eps=EPS, store_stats=True)
    buffers = _make_backward_buffers(x, w, group_size=1)
    dw_expected = torch.sum(dy * x * rstd[:, None], dim=0)
    first = None
    for _ in range(10):
        buffers.locks.zero_()
        _launch_backward_stage1(dy, x, w, rstd, buffers)
        torch.cuda.synchronize()
        assert buffers.locks.cpu().tolist() == [0, 1]
        _launch_backward_stage2(buffers, cols)
        torch.cuda.synchronize()
        assert_relative_frobenius(buffers.dw, dw_expected, max_relative_error=1e-2)
        if first is None:
            first = buffers.dw.clone()
        else:
            assert bits_equal(buffers.dw, first)


def test_counts_mark_only_active_groups() -> None:
    torch.manual_seed(4)
    x = torch.randn(5, 64, device="cuda")
    w = torch.randn(64, device="cuda")
    rstd = torch.empty(5, device="cuda")
    out = torch.empty_like(x)
    _launch_forward(x, w, out, rstd, eps=EPS, store_stats=True)
    buffers = _make_backward_buffers(x, w, group_size=8)
    _launch_backward_stage1(torch.randn_like(x), x, w, rstd, buffers)
    torch.cuda.synchronize()
    assert buffers.locks.cpu().tolist() == [0] * 8 + [1] * 5 + [0] * 3


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [1, 7, 64, 1000, 4096, 8192, 16384])
def test_forward_and_backward_match_the_oracle(dtype: torch.dtype, cols: int) -> None:
    if cols * torch.empty((), dtype=dtype).element_size() > 65536:
        pytest.skip("beyond the fused row budget")
    torch.manual_seed(cols)
    rows = 300
    x = torch.randn(rows, cols, device="cuda", dtype=dtype)
    w = (1 + 0.02 * torch.randn(cols, device="cuda")).to(dtype)
    dy = torch.randn(rows, cols, device="cuda", dtype=dtype)
    y = torch.empty_like(x)
    rstd = torch.empty(rows, device="cuda")
    _launch_forward(x, w, y, rstd, eps=1e-6, store_stats=True)
    _, y_ref, rstd_ref = oracle.rmsnorm_fwd(host(x), host(w), 1e-6, name(dtype))
    # FP32 statistics: relative 1e-5; stored outputs: the dtype table.
    torch.testing.assert_close(rstd, dev(rstd_ref, rstd), rtol=1e-5, atol=0)
    assert_close(y, dev(y_ref, y))
    buffers = _make_backward_buffers(x, w)
    _launch_backward_stage1(dy, x, w, rstd, buffers)
    _launch_backward_stage2(buffers, cols)
    dx_ref, dw_ref = oracle.rmsnorm_bwd(host(dy), host(x), host(w), host(rstd), name(dtype))
    assert_close(buffers.dx, dev(dx_ref, buffers.dx))
    assert_relative_frobenius(buffers.dw, dev(dw_ref, buffers.dw), max_relative_error=1e-2)
    if dtype == torch.float32:
        assert_relative_frobenius(buffers.dw, dev(dw_ref, buffers.dw), max_relative_error=1e-5)


@pytest.mark.parametrize("rows", [1, 300, 1030, 1537])
@pytest.mark.parametrize("dtype,cols", [(torch.bfloat16, 4096), (torch.float32, 1000)])
def test_stage1_ragged_and_empty_groups(rows: int, dtype: torch.dtype, cols: int) -> None:
    """512 groups over row counts below, at and above the group count: groups own
    the rows row % 512 == g, so 1030 rows give groups 0-5 three rows and the rest
    two, and a single row leaves one active group; the bf16 4096-column case takes
    the pipelined three-row loop."""
    torch.manual_seed(rows)
    x = torch.randn(rows, cols, device="cuda", dtype=dtype)
    w = (1 + 0.02 * torch.randn(cols, device="cuda")).to(dtype)
    dy = torch.randn(rows, cols, device="cuda", dtype=dtype)
    rstd = torch.empty(rows, device="cuda")
    _launch_forward(x, w, torch.empty_like(x), rstd, eps=1e-6, store_stats=True)
    buffers = _make_backward_buffers(x, w, group_size=512)
    _launch_backward_stage1(dy, x, w, rstd, buffers)
    _launch_backward_stage2(buffers, cols)
    torch.cuda.synchronize()
    dx_ref, dw_ref = oracle.rmsnorm_bwd(host(dy), host(x), host(w), host(rstd), name(dtype))
    assert_close(buffers.dx, dev(dx_ref, buffers.dx))
    assert_relative_frobenius(buffers.dw, dev(dw_ref, buffers.dw), max_relative_error=1e-2)


def test_backward_rejects_deterministic_mode_like_the_reference() -> None:
    """Reference ``tests/test_rms_norm.py:127-139``: RuntimeError "not deterministic"."""
    x, w, dy = _problem(rows=8, cols=16)
    previous = torch.are_deterministic_algorithms_enabled()
    previous_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        output = rms_norm(x, w)
        with pytest.raises(RuntimeError, match="not deterministic"):
            torch.autograd.grad(output, (x, w), grad_outputs=dy)
    finally:
        torch.use_deterministic_algorithms(previous, warn_only=previous_warn)


def test_backward_warns_in_deterministic_warn_only_mode_like_the_reference() -> None:
    """Reference ``tests/test_rms_norm.py:142-152``: RuntimeWarning "not deterministic"."""
    x, w, dy = _problem(rows=8, cols=16)
    previous = torch.are_deterministic_algorithms_enabled()
    previous_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True, warn_only=True)
        output = rms_norm(x, w)
        with pytest.warns(RuntimeWarning, match="not deterministic"):
            torch.autograd.grad(output, (x, w), grad_outputs=dy)
    finally:
        torch.use_deterministic_algorithms(previous, warn_only=previous_warn)


def test_backward_is_bitwise_reproducible_and_runs_in_deterministic_mode_when_allowed(
    monkeypatch: pytest.MonkeyPatch,
) -> None:
    monkeypatch.setattr(_norm_common, "REJECT_DETERMINISTIC_MODE", False)
    torch.manual_seed(5)
    x, w, dy = _problem(rows=515, cols=4096)
    previous = torch.are_deterministic_algorithms_enabled()
    previous_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        grads = []
        for _ in range(3):
            x2 = x.detach().requires_grad_(True)
            w2 = w.detach().requires_grad_(True)
            grads.append(torch.autograd.grad(rms_norm(x2, w2), (x2, w2), grad_outputs=dy))
    finally:
        torch.use_deterministic_algorithms(previous, warn_only=previous_warn)
    for dx, dw in grads[1:]:
        assert bits_equal(dx, grads[0][0])
        assert bits_equal(dw, grads[0][1])


def test_no_grad_forward_skips_statistics() -> None:
    torch.manual_seed(6)
    x = torch.randn(8, 256, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(256, device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        y = rms_norm(x, w)
    assert_close(y, F.rms_norm(x.float(), (256,), w.float(), EPS))
