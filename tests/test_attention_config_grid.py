"""GPU parity of the attention backward at benchmark config 5's own grid, and with batch > 1.

Config 5: Q/K/V bf16 [4, 32, N, D], N 8192 causal / 4096 non-causal, D 128 and 64, scale
1/sqrt(D), upstream dO ~ N(0, 1). The backward runs through the public autograd entry points
(`attention_causal` / `attention_noncausal`, reference `flash_attention.py:610-696`) over the
full grid, so batch strides and the heavy-first / XCD-interleaved tile schedule of every kernel
(preprocess, dK/dV, dQ) are exercised at the benchmarked shape. Sampled (batch, head) pairs with
batch > 0 are compared with the float32 gradient algebra (relative Frobenius 1e-2, the
attention bound of the multi-head tests); every head must be finite.

At small N, batched problems (batch 2-3) are compared with the CPU oracle
(`oracle.attn_bwd`, restating reference `flash_attention.py:383-395,437-466,512-533`), for both
head dims, both dtypes and both masks, plus grouped-query attention with batch 2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.flash_attention import (
    _launch_backward,
    _launch_forward,
    attention_causal,
    attention_noncausal,
    grouped_query_attention,
)

pytestmark = pytest.mark.gpu

SAMPLED_HEADS = [(0, 0), (0, 22), (1, 9), (1, 17), (2, 5), (2, 28), (3, 14), (3, 31)]


def _algebra32_head(q, k, v, do, causal):
    """dQ, dK, dV of one head [N, D] of softmax(QK^T/sqrt(d))V, in float32 on the GPU."""
    qf, kf, vf, dof = (t.detach().float() for t in (q, k, v, do))
    scale = q.shape[-1] ** -0.5
    s = torch.matmul(qf, kf.t().contiguous()) * scale
    if causal:
        n = q.shape[-2]
        s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool, device=q.device), 1), -torch.inf)
    p = torch.softmax(s, dim=-1)
    del s
    o = torch.matmul(p, vf)
    dv = torch.matmul(p.t().contiguous(), dof)
    dp = torch.matmul(dof, vf.t().contiguous())
    ds = p * (dp - (dof * o).sum(-1, keepdim=True))
    del p, dp
    dq = torch.matmul(ds, kf) * scale
    dk = torch.matmul(ds.t().contiguous(), qf) * scale
    return o, dq, dk, dv


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("causal", [True, False])
def test_config5_backward_on_the_full_grid(d, causal) -> None:
    b, h = 4, 32
    n = 8192 if causal else 4096
    print(f"config5 grid: B{b} H{h} N{n} D{d} causal={causal}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(500 + d + int(causal))
    shape = (b, h, n, d)
    q, k, v, do = (torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=g) for _ in range(4))
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    out = (attention_causal if causal else attention_noncausal)(*leaves)
    dq, dk, dv = torch.autograd.grad(out, leaves, grad_outputs=do)
    for grad in (out, dq, dk, dv):
        per_head = torch.isfinite(grad).flatten(2).all(-1)
        assert bool(per_head.all()), f"non-finite heads: {(~per_head).nonzero().tolist()[:8]}"
    for bi, hi in SAMPLED_HEADS:
        o_ref, *grads_ref = _algebra32_head(q[bi, hi], k[bi, hi], v[bi, hi], do[bi, hi], causal)
        assert_relative_frobenius(out[bi, hi], o_ref, max_relative_error=1e-2)
        for got, want in zip((dq, dk, dv), grads_ref):
            assert_relative_frobenius(got[bi, hi], want, max_relative_error=1e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize(("b", "h", "n"), [(2, 3, 77), (3, 2, 200)])
def test_batched_backward_matches_the_oracle(dtype, d, causal, b, h, n) -> None:
    torch.manual_seed(7 * n + d + int(causal) + b)
    shape = (b, h, n, d)
    q, k, v, do = (torch.randn(shape, device="cuda", dtype=dtype) for _ in range(4))
    out = torch.empty_like(q)
    lse = torch.empty(shape[:-1], device="cuda", dtype=torch.float32)
    _launch_forward(q, k, v, out, lse, causal=causal, store_lse=True)
    dq, dk, dv = _launch_backward(q, k, v, out, lse, do, causal=causal)
    o_ref, lse_ref = oracle.attn_fwd(host(q), host(k), host(v), d ** -0.5, causal, name(dtype))
    assert_close(out, dev(o_ref, out))
    torch.testing.assert_close(lse, dev(lse_ref, lse), rtol=1e-5, atol=1e-5)
    refs = oracle.attn_bwd(
        host(q), host(k), host(v), host(out), host(do), host(lse), d ** -0.5, causal, name(dtype)
    )
    for g, r in zip((dq, dk, dv), refs):
        for bi in range(b):
            assert_relative_frobenius(g[bi], dev(r[bi], g), max_relative_error=1e-2)
        assert_close(g, dev(r, g), rtol=5e-2, atol=5e-2)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [64, 128])
def test_batched_gqa_backward_matches_the_oracle(causal, d) -> None:
    b, hkv, group, n = 2, 2, 4, 200
    gen = torch.Generator(device="cuda").manual_seed(900 + d + int(causal))
    q = torch.randn(b, hkv * group, n, d, device="cuda", dtype=torch.bfloat16, generator=gen)
    k, v = (torch.randn(b, hkv, n, d, device="cuda", dtype=torch.bfloat16, generator=gen) for _ in range(2))
    do = torch.randn_like(q)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    out = grouped_query_attention(*leaves, causal=causal)
    dq, dk, dv = torch.autograd.grad(out, leaves, grad_outputs=do)
    kr, vr = (np.repeat(host(t), group, axis=1) for t in (k, v))
    scale = d ** -0.5
    o_ref, lse_ref = oracle.attn_fwd(host(q), kr, vr, scale, causal, "bfloat16")
    assert_close(out, dev(o_ref, out))
    dq_ref, dk_rep, dv_rep = oracle.attn_bwd(host(q), kr, vr, o_ref, host(do), lse_ref, scale, causal, "bfloat16")
    dk_ref = dk_rep.reshape(b, hkv, group, n, d).astype(np.float64).sum(axis=2).astype(np.float32)
    dv_ref = dv_rep.reshape(b, hkv, group, n, d).astype(np.float64).sum(axis=2).astype(np.float32)
    for bi in range(b):
        assert_relative_frobenius(dq[bi], dev(dq_ref[bi], dq), max_relative_error=1e-2)
        assert_relative_frobenius(dk[bi], dev(dk_ref[bi], dk), max_relative_error=1e-2)
        assert_relative_frobenius(dv[bi], dev(dv_ref[bi], dv), max_relative_error=1e-2)
