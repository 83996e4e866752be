"""GPU parity of grouped-query attention (tk_attn_fwd_gqa, tk_attn_bwd_dkdv_gqa,
tk_attn_bwd_dq_gqa).

References: the CPU oracle's multi-head attention on K/V repeated per group (the
forward and dQ are exactly that; dK and dV are its per-query-head gradients summed
over each group), the float32 gradient algebra, and the library's own multi-head
kernels, which GQA with kv_heads == heads must reproduce bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits_equal, dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.flash_attention import attention_causal, grouped_query_attention

pytestmark = pytest.mark.gpu


def _inputs(b, h, hkv, n, d, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(b, h, n, d, device="cuda", dtype=dtype, generator=g)
    k = torch.randn(b, hkv, n, d, device="cuda", dtype=dtype, generator=g)
    v = torch.randn(b, hkv, n, d, device="cuda", dtype=dtype, generator=g)
    do = torch.randn(b, h, n, d, device="cuda", dtype=dtype, generator=g)
    return q, k, v, do


def _grads(q, k, v, do, causal):
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    out = grouped_query_attention(*leaves, causal=causal)
    out.backward(do)
    return out.detach(), leaves[0].grad, leaves[1].grad, leaves[2].grad


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [2, 4, 8])
def test_forward_and_backward_match_the_oracle(causal, d, group) -> None:
    b, hkv, n = 1, 2, 200  # ragged: 200 is not a multiple of the 64-row blocks
    q, k, v, do = _inputs(b, hkv * group, hkv, n, d, torch.bfloat16, seed=group * 10 + d + causal)
    o, dq, dk, dv = _grads(q, k, v, do, causal)
    kr = np.repeat(host(k), group, axis=1)
    vr = np.repeat(host(v), group, axis=1)
    scale = d ** -0.5
    o_ref, lse_ref = oracle.attn_fwd(host(q), kr, vr, scale, causal, name(q.dtype))
    assert_close(o, dev(o_ref, o))
    dq_ref, dk_rep, dv_rep = oracle.attn_bwd(host(q), kr, vr, o_ref, host(do), lse_ref, scale,
                                             causal, name(q.dtype))
    dk_ref = dk_rep.reshape(b, hkv, group, n, d).astype(np.float64).sum(axis=2)
    dv_ref = dv_rep.reshape(b, hkv, group, n, d).astype(np.float64).sum(axis=2)
    # The tolerances of the multi-head backward tests (relative Frobenius 1e-2).
    assert_relative_frobenius(dq, dev(dq_ref, dq), max_relative_error=1e-2)
    assert_relative_frobenius(dk, dev(dk_ref.astype(np.float32), dk), max_relative_error=1e-2)
    assert_relative_frobenius(dv, dev(dv_ref.astype(np.float32), dv), max_relative_error=1e-2)


def test_one_head_per_group_is_bitwise_multi_head_attention() -> None:
    q, k, v, do = _inputs(2, 4, 4, 333, 128, torch.bfloat16, seed=5)
    o, dq, dk, dv = _grads(q, k, v, do, True)
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    ref = attention_causal(*leaves)
    ref.backward(do)
    assert bits_equal(o, ref.detach())
    for got, want in zip((dq, dk, dv), leaves):
        assert bits_equal(got, want.grad)


def test_matches_float32_gradient_algebra_at_a_larger_shape() -> None:
    b, h, hkv, n, d = 1, 8, 2, 1024, 128
    q, k, v, do = _inputs(b, h, hkv, n, d, torch.bfloat16, seed=6)
    o, dq, dk, dv = _grads(q, k, v, do, True)
    group = h // hkv
    qf, kf, vf, dof = (t.float() for t in (q, k, v, do))
    kr = kf.repeat_interleave(group, dim=1).contiguous()
    vr = vf.repeat_interleave(group, dim=1).contiguous()
    s = torch.matmul(qf, kr.transpose(-2, -1).contiguous()) * d ** -0.5
    s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool, device="cuda"), 1), -torch.inf)
    p = torch.softmax(s, dim=-1)
    o32 = torch.matmul(p, vr)
    dv32 = torch.matmul(p.transpose(-2, -1).contiguous(), dof)
    dp = torch.matmul(dof, vr.transpose(-2, -1).contiguous())
    ds = p * (dp - (dof * o32).sum(-1, keepdim=True))
    dq32 = torch.matmul(ds, kr) * d ** -0.5
    dk32 = torch.matmul(ds.transpose(-2, -1).contiguous(), qf) * d ** -0.5
    dk32 = dk32.reshape(b, hkv, group, n, d).sum(2)
    dv32 = dv32.reshape(b, hkv, group, n, d).sum(2)
    assert_relative_frobenius(o, o32, max_relative_error=1e-2)
    for got, want in ((dq, dq32), (dk, dk32), (dv, dv32)):
        assert_relative_frobenius(got, want, max_relative_error=1e-2)


def test_backward_is_bitwise_reproducible() -> None:
    q, k, v, do = _inputs(1, 8, 2, 500, 64, torch.float16, seed=7)
    first = _grads(q, k, v, do, False)
    second = _grads(q, k, v, do, False)
    for a, b in zip(first, second):
        assert bits_equal(a, b)


def test_inference_skips_the_lse() -> None:
    q, k, v, _ = _inputs(1, 8, 4, 100, 64, torch.bfloat16, seed=8)
    with torch.no_grad():
        o = grouped_query_attention(q, k, v, causal=True)
    kr, vr = (np.repeat(host(t), 2, axis=1) for t in (k, v))
    o_ref, _ = oracle.attn_fwd(host(q), kr, vr, 64 ** -0.5, True, name(q.dtype))
    assert_close(o, dev(o_ref, o))


def test_contract() -> None:
    q = torch.empty(1, 6, 64, 64, device="cuda", dtype=torch.bfloat16)
    k = torch.empty(1, 4, 64, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="multiple of the K/V heads"):
        grouped_query_attention(q, k, k, causal=True)
    with pytest.raises(ValueError, match="agree on batch"):
        grouped_query_attention(q, k[:, :, :32], k[:, :, :32], causal=True)
