"""GPU parity of rotate-half RoPE forward/backward.

Reference cases follow the reference's tests/test_rope.py (seeds 40-43,
strides 2/3/4, 1e-7 bounds, the inverse-rotation and norm identities). RoPE
has no transcendental: with separately rounded products the kernel and the
oracle compute the same float32 operations, so those comparisons are bitwise.
"""

from __future__ import annotations

import math

import pytest
import torch

from _helpers import bits_equal, dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_relative_frobenius
from tklab.kernels.rope import _launch_backward, rope

pytestmark = pytest.mark.gpu


def _rotate_half(x, cos, sin):
    a, b = x.chunk(2, dim=-1)
    return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)


def _problem(rows: int = 37, cols: int = 1000):
    x = torch.randn(rows * 2, cols, device="cuda")[::2].detach().requires_grad_(True)
    dy = torch.randn(rows * 3, cols, device="cuda")[::3]
    angles = torch.randn(rows * 4, cols // 2, device="cuda")[::4]
    cos = torch.cos(angles).detach().requires_grad_(True)
    sin = torch.sin(angles).detach().requires_grad_(True)
    return x, cos, sin, dy


def test_forward_matches_rotate_half() -> None:
    torch.manual_seed(40)
    x, cos, sin, _ = _problem()
    assert_relative_frobenius(rope(x, cos, sin), _rotate_half(x, cos, sin), max_relative_error=1e-7)


def test_gradients_match_autograd() -> None:
    torch.manual_seed(41)
    x, cos, sin, dy = _problem(rows=67)
    refs = torch.autograd.grad(_rotate_half(x, cos, sin), (x, cos, sin), grad_outputs=dy)
    leaves = [t.detach().requires_grad_(True) for t in (x, cos, sin)]
    got = torch.autograd.grad(rope(*leaves), leaves, grad_outputs=dy)
    for a, b in zip(got, refs):
        assert_relative_frobenius(a, b, max_relative_error=1e-7)


def test_x_gradient_is_the_inverse_rotation() -> None:
    torch.manual_seed(42)
    x, cos, sin, dy = _problem(rows=17, cols=128)
    (dx,) = torch.autograd.grad(rope(x, cos, sin), (x,), grad_outputs=dy)
    assert_relative_frobenius(dx, _rotate_half(dy, cos, -sin), max_relative_error=1e-7)


def test_rotation_preserves_row_norms() -> None:
    torch.manual_seed(43)
    x, cos, sin, _ = _problem(rows=17, cols=128)
    y = rope(x, cos, sin)
    torch.testing.assert_close((y * y).sum(-1), (x * x).sum(-1), rtol=1e-5, atol=1e-5)


def test_only_requested_table_gradients_are_computed() -> None:
    torch.manual_seed(44)
    x, cos, sin, dy = _problem(rows=9, cols=64)
    cos2 = cos.detach()
    dx, dsin = torch.autograd.grad(rope(x, cos2, sin), (x, sin), grad_outputs=dy)
    refs = torch.autograd.grad(_rotate_half(x, cos2, sin), (x, sin), grad_outputs=dy)
    assert_relative_frobenius(dx, refs[0], max_relative_error=1e-7)
    assert_relative_frobenius(dsin, refs[1], max_relative_error=1e-7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [2, 6, 64, 128, 1000, 2048])
def test_bitwise_against_the_oracle(dtype: torch.dtype, cols: int) -> None:
    torch.manual_seed(cols)
    rows = 41
    x = torch.randn(rows, cols, device="cuda", dtype=dtype)
    angles = torch.randn(rows, cols // 2, device="cuda")
    cos, sin = torch.cos(angles).to(dtype), torch.sin(angles).to(dtype)
    dy = torch.randn_like(x)
    y = rope(x, cos, sin)
    dx, dcos, dsin = _launch_backward(dy, x, cos, sin)
    n = name(dtype)
    assert bits_equal(y, dev(oracle.rope_fwd(host(x), host(cos), host(sin), n), y).to(dtype))
    refs = oracle.rope_bwd(host(dy), host(x), host(cos), host(sin), n)
    for got, want in zip((dx, dcos, dsin), refs):
        assert bits_equal(got, dev(want, got).to(dtype))


def test_config_shape_bf16_q_4x32x4096x128() -> None:
    """benchmark config 3 RoPE: q [4,32,4096,128] bf16 as [524288, 128], base 1e4, positions 0..4095."""
    torch.manual_seed(0)
    b, h, s, d = 4, 32, 4096, 128
    q = torch.randn(b, h, s, d, device="cuda", dtype=torch.bfloat16)
    inv_freq = 10000.0 ** (-torch.arange(0, d, 2, device="cuda", dtype=torch.float32) / d)
    angle = torch.arange(s, device="cuda", dtype=torch.float32)[:, None] * inv_freq[None, :]
    cos = torch.cos(angle).to(torch.bfloat16).expand(b * h, s, d // 2).reshape(-1, d // 2)
    sin = torch.sin(angle).to(torch.bfloat16).expand(b * h, s, d // 2).reshape(-1, d // 2)
    x = q.view(-1, d)
    y = rope(x, cos, sin)
    rows = torch.arange(0, x.shape[0], 509, device="cuda")
    want = oracle.rope_fwd(host(x[rows]), host(cos[rows]), host(sin[rows]), "bfloat16")
    assert bits_equal(y[rows], dev(want, y).to(torch.bfloat16))
    norms_in = x.float().pow(2).sum(-1)
    norms_out = y.float().pow(2).sum(-1)
    # bf16 tables: |cos^2 + sin^2 - 1| <= ~2^-7; outputs round to bf16 too.
    assert torch.allclose(norms_out, norms_in, rtol=2e-2, atol=1e-2)
    assert math.isfinite(float(y.float().abs().max()))


def _config3_tables(b: int, h: int, s: int, d: int):
    inv_freq = 10000.0 ** (-torch.arange(0, d, 2, device="cuda", dtype=torch.float32) / d)
    angle = torch.arange(s, device="cuda", dtype=torch.float32)[:, None] * inv_freq[None, :]
    cos = torch.cos(angle).to(torch.bfloat16).expand(b * h, s, d // 2).reshape(-1, d // 2)
    sin = torch.sin(angle).to(torch.bfloat16).expand(b * h, s, d // 2).reshape(-1, d // 2)
    return cos, sin


def test_config_shape_backward_bf16_4x32x4096x128() -> None:
    """benchmark config 3 RoPE backward: dx only (constant tables, the autograd path) and the
    dcos/dsin variant, at [4,32,4096,128] bf16, bitwise on every 509th row against the oracle;
    dx is the inverse rotation of dy, so row norms are preserved up to bf16 rounding."""
    torch.manual_seed(1)
    b, h, s, d = 4, 32, 4096, 128
    cos, sin = _config3_tables(b, h, s, d)
    x = torch.randn(b * h * s, d, device="cuda", dtype=torch.bfloat16).requires_grad_(True)
    dy = torch.randn_like(x)
    (dx,) = torch.autograd.grad(rope(x, cos, sin), (x,), grad_outputs=dy)
    rows = torch.arange(0, x.shape[0], 509, device="cuda")
    want_dx, want_dcos, want_dsin = oracle.rope_bwd(
        host(dy[rows]), host(x[rows]), host(cos[rows]), host(sin[rows]), "bfloat16"
    )
    assert bits_equal(dx[rows], dev(want_dx, dx).to(torch.bfloat16))
    assert torch.allclose(dx.float().pow(2).sum(-1), dy.float().pow(2).sum(-1), rtol=2e-2, atol=1e-2)
    dx_all, dcos, dsin = _launch_backward(dy, x.detach(), cos, sin)
    assert bits_equal(dx_all, dx)
    assert bits_equal(dcos[rows], dev(want_dcos, dcos).to(torch.bfloat16))
    assert bits_equal(dsin[rows], dev(want_dsin, dsin).to(torch.bfloat16))
