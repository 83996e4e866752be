"""GPU tests of the registry kernels outside the hot path: vector_add,
activations and LayerNorm (forward and backward against PyTorch autograd on
float32 upcasts, lock/count state, determinism)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from _helpers import bits_equal
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.activations import gelu, relu, silu, tanh
from tklab.kernels.layer_norm import (
    _launch_backward_stage1,
    _launch_backward_stage2,
    _launch_forward,
    _make_backward_buffers,
    layer_norm,
)
from tklab.kernels.vector_add import vector_add

pytestmark = pytest.mark.gpu

ACTIVATIONS = [(relu, torch.relu), (gelu, F.gelu), (silu, F.silu), (tanh, torch.tanh)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [1, 7, 1009, 4096, 1 << 20])
def test_vector_add(dtype, n) -> None:
    torch.manual_seed(n)
    x = torch.randn(n, device="cuda", dtype=dtype)
    y = torch.randn(n, device="cuda", dtype=dtype)
    assert bits_equal(vector_add(x, y), x + y)


def test_vector_add_strided_and_broadcast() -> None:
    torch.manual_seed(1)
    x = torch.randn(2018, device="cuda")[::2]
    y = torch.randn(3027, device="cuda")[::3]
    assert bits_equal(vector_add(x, y), x + y)
    b = torch.randn(1, device="cuda").expand(1009)
    assert bits_equal(vector_add(x, b), x + b)


@pytest.mark.parametrize(("ours", "theirs"), ACTIVATIONS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_activation_forward_and_backward(ours, theirs, dtype) -> None:
    torch.manual_seed(7)
    x = torch.randn(67 * 2, 1000, device="cuda", dtype=dtype)[::2].detach().requires_grad_(True)
    dy = torch.randn(67, 1000, device="cuda", dtype=dtype)
    x32 = x.detach().float().requires_grad_(True)
    ref = theirs(x32)
    (dref,) = torch.autograd.grad(ref, (x32,), grad_outputs=dy.float())
    out = ours(x)
    (dx,) = torch.autograd.grad(out, (x,), grad_outputs=dy)
    bound = 1e-6 if dtype == torch.float32 else 1e-2
    assert_relative_frobenius(out, ref, max_relative_error=bound)
    assert_relative_frobenius(dx, dref, max_relative_error=max(bound, 1e-5))


@pytest.mark.parametrize(("ours", "theirs"), ACTIVATIONS)
def test_activation_extremes_stay_finite(ours, theirs) -> None:
    x = torch.tensor([[-100.0, -80.0, -20.0, -1.0, 0.0, 1.0, 20.0, 100.0]], device="cuda")
    x = x.repeat(4, 1).requires_grad_(True)
    out = ours(x)
    (dx,) = torch.autograd.grad(out, (x,), grad_outputs=torch.ones_like(out))
    assert torch.isfinite(out).all() and torch.isfinite(dx).all()
    torch.testing.assert_close(out, theirs(x.detach()), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cols", [1, 1000, 4096, 8192])
def test_layer_norm_forward_and_gradients(dtype, cols) -> None:
    torch.manual_seed(cols)
    rows = 67
    x = torch.randn(rows * 2, cols, device="cuda", dtype=dtype)[::2].detach().requires_grad_(True)
    w = torch.randn(cols, device="cuda", dtype=dtype, requires_grad=True)
    b = torch.randn(cols, device="cuda", dtype=dtype, requires_grad=True)
    dy = torch.randn(rows, cols, device="cuda", dtype=dtype)
    leaves32 = [t.detach().float().requires_grad_(True) for t in (x, w, b)]
    ref = F.layer_norm(leaves32[0], (cols,), leaves32[1], leaves32[2], 1e-5)
    refs = torch.autograd.grad(ref, leaves32, grad_outputs=dy.float())
    out = layer_norm(x, w, b)
    got = torch.autograd.grad(out, (x, w, b), grad_outputs=dy)
    bound = 1e-4 if dtype == torch.float32 else 1e-2
    assert_relative_frobenius(out, ref, max_relative_error=bound)
    if cols > 1:  # a single column normalizes to exactly zero: dx is pure rounding noise
        for g, r in zip(got, refs):
            assert_relative_frobenius(g, r, max_relative_error=max(bound, 1e-3))


def test_layer_norm_single_group_state_and_repeatability() -> None:
    torch.manual_seed(9)
    rows, cols = 1025, 1000
    x = torch.randn(rows, cols, device="cuda")
    w = torch.randn(cols, device="cuda")
    b = torch.randn(cols, device="cuda")
    dy = torch.randn(rows, cols, device="cuda")
    out = torch.empty_like(x)
    mean = torch.empty(rows, device="cuda")
    rstd = torch.empty(rows, device="cuda")
    _launch_forward(x, w, b, out, mean, rstd, eps=1e-5, store_stats=True)
    assert_close(mean, x.mean(dim=1))
    buffers = _make_backward_buffers(x, w, group_size=1)
    first = None
    for _ in range(3):
        buffers.locks.zero_()
        _launch_backward_stage1(dy, x, w, mean, rstd, buffers)
        torch.cuda.synchronize()
        assert buffers.locks.cpu().tolist() == [0, 1]
        _launch_backward_stage2(buffers, cols)
        x_hat = (x - mean[:, None]) * rstd[:, None]
        assert_relative_frobenius(buffers.dw, (dy * x_hat).sum(0), max_relative_error=1e-4)
        assert_relative_frobenius(buffers.db, dy.sum(0), max_relative_error=1e-4)
        if first is None:
            first = (buffers.dw.clone(), buffers.db.clone())
        else:
            assert bits_equal(buffers.dw, first[0]) and bits_equal(buffers.db, first[1])
