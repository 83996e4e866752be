"""GPU parity of SwiGLU forward/backward.

Reference cases follow the reference's tests/test_swiglu.py (seeds 30-31,
strides 2/3/4, the 1e-6 relative-Frobenius bound, extreme gates); oracle
comparisons across dtypes and at the config shape are this build's own.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from _helpers import dev, host, name, strided_rows
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.swiglu import _launch_backward, swiglu

pytestmark = pytest.mark.gpu


def _problem(rows: int = 37, cols: int = 1000):
    value = strided_rows(rows, cols, 2, requires_grad=True)
    gate = strided_rows(rows, cols, 3, requires_grad=True)
    dy = strided_rows(rows, cols, 4)
    return value, gate, dy


def test_forward_matches_pytorch_on_strided_tail() -> None:
    torch.manual_seed(30)
    value, gate, _ = _problem()
    assert_relative_frobenius(swiglu(value, gate), value * F.silu(gate), max_relative_error=1e-6)


def test_gradients_match_autograd() -> None:
    torch.manual_seed(31)
    value, gate, dy = _problem(rows=67)
    refs = torch.autograd.grad(value * F.silu(gate), (value, gate), grad_outputs=dy)
    v2, g2 = value.detach().requires_grad_(True), gate.detach().requires_grad_(True)
    got = torch.autograd.grad(swiglu(v2, g2), (v2, g2), grad_outputs=dy)
    for a, b in zip(got, refs):
        assert_relative_frobenius(a, b, max_relative_error=1e-6)


def test_extreme_gates_stay_finite() -> None:
    value = torch.randn(4, 8, device="cuda", requires_grad=True)
    gate = torch.tensor([-100.0, -80.0, -20.0, -1.0, 0.0, 1.0, 20.0, 100.0], device="cuda")
    gate = gate.repeat(4, 1).requires_grad_(True)
    out = swiglu(value, gate)
    dv, dg = torch.autograd.grad(out, (value, gate), grad_outputs=torch.ones_like(out))
    for t in (out, dv, dg):
        assert torch.isfinite(t).all()
    assert_relative_frobenius(out, value * F.silu(gate), max_relative_error=1e-6)


def test_backward_runs_in_deterministic_mode() -> None:
    previous = torch.are_deterministic_algorithms_enabled()
    previous_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        value, gate, dy = _problem(rows=17, cols=128)
        torch.autograd.grad(swiglu(value, gate), (value, gate), grad_outputs=dy)
    finally:
        torch.use_deterministic_algorithms(previous, warn_only=previous_warn)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [1, 5, 8, 1000, 14336])
def test_matches_the_oracle(dtype: torch.dtype, cols: int) -> None:
    torch.manual_seed(cols)
    value = torch.randn(33, cols, device="cuda", dtype=dtype)
    gate = torch.randn(33, cols, device="cuda", dtype=dtype)
    dy = torch.randn(33, cols, device="cuda", dtype=dtype)
    y = swiglu(value, gate)
    dv, dg = _launch_backward(dy, value, gate)
    n = name(dtype)
    assert_close(y, dev(oracle.swiglu_fwd(host(value), host(gate), n), y))
    dv_ref, dg_ref = oracle.swiglu_bwd(host(dy), host(value), host(gate), n)
    assert_close(dv, dev(dv_ref, dv))
    assert_close(dg, dev(dg_ref, dg))


def test_config_shape_bf16_16384x14336() -> None:
    """benchmark config 3 SwiGLU: gate, up ~N(0,1) [16384, 14336] bf16; every 97th row checked."""
    torch.manual_seed(0)
    gate = torch.randn(16384, 14336, device="cuda", dtype=torch.bfloat16)
    up = torch.randn(16384, 14336, device="cuda", dtype=torch.bfloat16)
    dy = torch.randn(16384, 14336, device="cuda", dtype=torch.bfloat16)
    y = swiglu(up, gate)
    dv, dg = _launch_backward(dy, up, gate)
    rows = torch.arange(0, 16384, 97, device="cuda")
    g, u, d = host(gate[rows]), host(up[rows]), host(dy[rows])
    assert_close(y[rows], dev(oracle.swiglu_fwd(u, g, "bfloat16"), y))
    dv_ref, dg_ref = oracle.swiglu_bwd(d, u, g, "bfloat16")
    assert_close(dv[rows], dev(dv_ref, dv))
    assert_close(dg[rows], dev(dg_ref, dg))
