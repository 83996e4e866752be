"""GPU parity of the attention backward (preprocess, dK/dV, dQ).

Reference checks (tests/test_flash_attention_backward.py of the reference):
gradients vs SDPA autograd within relative Frobenius 3e-2 for (1, 16, N, 64)
float16 at N = 128 and 1000 (seeds 41 + N + causal), and vs the float32
gradient algebra within 1e-3 at N = 128 (seeds 79 + causal). References run
on float32 upcasts. This build adds the CPU oracle and a per-head float32
check at a benchmark-sized head.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from _helpers import dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.flash_attention import (
    _launch_backward,
    _launch_forward,
    attention_causal,
    attention_noncausal,
)

pytestmark = pytest.mark.gpu

KERNELS = [(False, attention_noncausal), (True, attention_causal)]


def _leaves(shape, dtype=torch.float16):
    q, k, v = (torch.randn(shape, device="cuda", dtype=dtype, requires_grad=True) for _ in range(3))
    do = torch.randn(shape, device="cuda", dtype=dtype)
    return q, k, v, do


def _algebra32(q, k, v, do, causal):
    """dQ, dK, dV of softmax(QK^T/sqrt(d)) V evaluated in float32."""
    qf, kf, vf, dof = (t.detach().float() for t in (q, k, v, do))
    scale = q.shape[-1] ** -0.5
    s = torch.matmul(qf, kf.transpose(-2, -1).contiguous()) * scale
    if causal:
        n = q.shape[-2]
        s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool, device="cuda"), 1), -torch.inf)
    p = torch.softmax(s, dim=-1)
    o = torch.matmul(p, vf)
    dv = torch.matmul(p.transpose(-2, -1).contiguous(), dof)
    dp = torch.matmul(dof, vf.transpose(-2, -1).contiguous())
    ds = p * (dp - (dof * o).sum(-1, keepdim=True))
    dq = torch.matmul(ds, kf) * scale
    dk = torch.matmul(ds.transpose(-2, -1).contiguous(), qf) * scale
    return dq, dk, dv


@pytest.mark.parametrize(("causal", "kernel"), KERNELS)
@pytest.mark.parametrize("n", [128, 1000])
def test_gradients_match_sdpa(causal, kernel, n) -> None:
    torch.manual_seed(41 + n + int(causal))
    q, k, v, do = _leaves((1, 16, n, 64))
    q32, k32, v32 = (t.detach().float().requires_grad_(True) for t in (q, k, v))
    ref = F.scaled_dot_product_attention(q32, k32, v32, is_causal=causal)
    refs = torch.autograd.grad(ref, (q32, k32, v32), grad_outputs=do.float())
    got = torch.autograd.grad(kernel(q, k, v), (q, k, v), grad_outputs=do)
    for g, r in zip(got, refs):
        assert torch.isfinite(g).all()
        assert_relative_frobenius(g, r, max_relative_error=3e-2)


@pytest.mark.parametrize(("causal", "kernel"), KERNELS)
def test_gradients_match_float32_algebra(causal, kernel) -> None:
    torch.manual_seed(79 + int(causal))
    q, k, v, do = _leaves((1, 16, 128, 64))
    expected = _algebra32(q, k, v, do, causal)
    got = torch.autograd.grad(kernel(q, k, v), (q, k, v), grad_outputs=do)
    for g, r in zip(got, expected):
        assert_relative_frobenius(g, r, max_relative_error=1e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [1, 77, 200, 385])
def test_matches_the_oracle(dtype, d, causal, n) -> None:
    torch.manual_seed(3 * n + d + int(causal))
    shape = (1, 3, n, d)
    q, k, v, do = (torch.randn(shape, device="cuda", dtype=dtype) for _ in range(4))
    out = torch.empty_like(q)
    lse = torch.empty(shape[:-1], device="cuda", dtype=torch.float32)
    _launch_forward(q, k, v, out, lse, causal=causal, store_lse=True)
    dq, dk, dv = _launch_backward(q, k, v, out, lse, do, causal=causal)
    refs = oracle.attn_bwd(
        host(q), host(k), host(v), host(out), host(do), host(lse), d ** -0.5, causal, name(dtype)
    )
    for g, r in zip((dq, dk, dv), refs):
        assert_relative_frobenius(g, dev(r, g), max_relative_error=1e-2)
        assert_close(g, dev(r, g), rtol=5e-2, atol=5e-2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_paired_key_blocks_on_the_xcd_path(dtype) -> None:
    """Causal head_dim 64 dK/dV deals key blocks i and NB-1-i to one workgroup: batch x heads
    a multiple of 8 (each XCD takes its eighth of the heads) and 3 blocks of 128 keys (the
    middle one has no partner), against the oracle."""
    torch.manual_seed(11)
    shape = (2, 4, 384, 64)
    q, k, v, do = (torch.randn(shape, device="cuda", dtype=dtype) for _ in range(4))
    out = torch.empty_like(q)
    lse = torch.empty(shape[:-1], device="cuda", dtype=torch.float32)
    _launch_forward(q, k, v, out, lse, causal=True, store_lse=True)
    dq, dk, dv = _launch_backward(q, k, v, out, lse, do, causal=True)
    refs = oracle.attn_bwd(
        host(q), host(k), host(v), host(out), host(do), host(lse), 64 ** -0.5, True, name(dtype)
    )
    for g, r in zip((dq, dk, dv), refs):
        assert_relative_frobenius(g, dev(r, g), max_relative_error=1e-2)
        assert_close(g, dev(r, g), rtol=5e-2, atol=5e-2)


def test_backward_is_bitwise_reproducible() -> None:
    torch.manual_seed(8)
    q, k, v, do = _leaves((2, 4, 640, 128), dtype=torch.bfloat16)
    runs = [torch.autograd.grad(attention_causal(q, k, v), (q, k, v), grad_outputs=do) for _ in range(3)]
    for grads in runs[1:]:
        for a, b in zip(grads, runs[0]):
            assert torch.equal(a, b)


@pytest.mark.parametrize("causal", [True, False])
def test_config_sized_head_matches_float32_algebra(causal) -> None:
    """benchmark config 5 per-head size (N 8192 causal / 4096 non-causal, D 128, bf16), 2 heads."""
    torch.manual_seed(0)
    n = 8192 if causal else 4096
    q, k, v, do = _leaves((1, 2, n, 128), dtype=torch.bfloat16)
    got = torch.autograd.grad(
        (attention_causal if causal else attention_noncausal)(q, k, v), (q, k, v), grad_outputs=do
    )
    for h in range(2):
        expected = _algebra32(q[:, h : h + 1], k[:, h : h + 1], v[:, h : h + 1], do[:, h : h + 1], causal)
        for g, r in zip(got, expected):
            assert_relative_frobenius(g[:, h : h + 1], r, max_relative_error=1e-2)
