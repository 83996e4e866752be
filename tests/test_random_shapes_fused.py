"""Seeded random-shape parity sweep over the fused and extension entry points.

The companion of ``test_random_shapes.py`` for variable-length attention (random
sequence lengths, empty sequences and padded packings), RoPE'd attention, the
SwiGLU-epilogue GEMM, the row-scaled RMSNorm GEMMs, LayerNorm, the activations
and vector_add. Each case draws its shape from a fixed seed and compares against
float32 PyTorch math at the storage dtype's tolerance (elementwise where the
kernel rounds once, relative Frobenius for gradients that sum rounded products).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels._norm_common import EPS
from tklab.kernels.activations import gelu, relu, silu, tanh
from tklab.kernels.flash_attention import rope_attention, varlen_attention
from tklab.kernels.layer_norm import layer_norm
from tklab.kernels.matmul_swiglu import matmul_swiglu
from tklab.kernels.rms_norm_matmul import fold_norm_weight, residual_rms_norm_matmul, rms_norm_matmul
from tklab.kernels.vector_add import vector_add

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]
CASES = range(6)


def _seeded(op: str, case: int) -> np.random.RandomState:
    """Shape generator of one case (seeded from the op's name bytes, not the salted hash)."""
    return np.random.RandomState(sum(op.encode()) * 100 + case + 7)


def _attention32(q, k, v, causal):
    """softmax(Q K^T / sqrt(d)) V in float32 for [b, h, n, d] leaves, K/V repeated per group."""
    group = q.shape[1] // k.shape[1]
    kr = k.repeat_interleave(group, dim=1)
    vr = v.repeat_interleave(group, dim=1)
    s = torch.matmul(q, kr.transpose(-2, -1).contiguous()) * q.shape[-1] ** -0.5
    if causal:
        n = q.shape[-2]
        s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool, device=q.device), 1), -torch.inf)
    return torch.matmul(torch.softmax(s, dim=-1), vr)


@pytest.mark.parametrize("case", range(8))
def test_varlen_attention_forward_and_backward(case: int) -> None:
    r = _seeded("varlen", case)
    nseq = int(r.randint(1, 6))
    lens = [int(x) for x in r.randint(0, 400, size=nseq)]
    if case % 3 == 0:
        lens[0] = 0  # an empty sequence
    if sum(lens) == 0:
        lens[-1] = 1 + int(r.randint(0, 100))
    pad = int(r.randint(0, 40)) if case % 2 else 0  # tokens past the last sequence
    kv_heads = int(r.randint(1, 3))
    group = int(r.choice([1, 2, 4]))
    d = int(r.choice([64, 128]))
    causal = bool(case % 2)
    dtype = DTYPES[(case // 2) % 2]
    heads = kv_heads * group
    total = sum(lens) + pad
    torch.manual_seed(case)
    q = torch.randn(total, heads, d, device="cuda", dtype=dtype, requires_grad=True)
    k = torch.randn(total, kv_heads, d, device="cuda", dtype=dtype, requires_grad=True)
    v = torch.randn(total, kv_heads, d, device="cuda", dtype=dtype, requires_grad=True)
    do = torch.randn(total, heads, d, device="cuda", dtype=dtype)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cu = torch.from_numpy(offsets).cuda()
    o = varlen_attention(q, k, v, cu, max(max(lens), 1), causal=causal)
    got = torch.autograd.grad(o, (q, k, v), grad_outputs=do)

    leaves = [t.detach().float().requires_grad_(True) for t in (q, k, v)]
    pieces = []
    for b in range(nseq):
        a, e = int(offsets[b]), int(offsets[b + 1])
        if e == a:
            continue
        qs, ks, vs = (t[a:e].transpose(0, 1).unsqueeze(0) for t in leaves)
        pieces.append((a, e, _attention32(qs, ks, vs, causal)[0].transpose(0, 1)))
    o_ref = torch.zeros(total, heads, d, device="cuda")
    for a, e, piece in pieces:
        o_ref[a:e] = piece.detach()
    loss = sum((piece * do[a:e].float()).sum() for a, e, piece in pieces)
    refs = torch.autograd.grad(loss, leaves, allow_unused=True) if pieces else (None,) * 3
    assert_close(o, o_ref)
    for g, ref in zip(got, refs):
        ref = torch.zeros_like(g, dtype=torch.float32) if ref is None else ref
        assert torch.isfinite(g).all()
        assert_relative_frobenius(g, ref, max_relative_error=1e-2)
        if pad:
            assert torch.count_nonzero(g[total - pad:]) == 0


@pytest.mark.parametrize("case", CASES)
def test_rope_attention_forward_and_backward(case: int) -> None:
    r = _seeded("rope_attention", case)
    batch = int(r.randint(1, 3))
    kv_heads = int(r.randint(1, 3))
    group = int(r.choice([1, 2, 4]))
    n = int(r.randint(1, 400))
    d = int(r.choice([64, 128]))
    causal = bool(case % 2)
    dtype = DTYPES[(case // 2) % 2]
    torch.manual_seed(case)
    q = torch.randn(batch, kv_heads * group, n, d, device="cuda", dtype=dtype, requires_grad=True)
    k = torch.randn(batch, kv_heads, n, d, device="cuda", dtype=dtype, requires_grad=True)
    v = torch.randn(batch, kv_heads, n, d, device="cuda", dtype=dtype, requires_grad=True)
    do = torch.randn_like(q)
    positions = n + int(r.randint(0, 50))
    inv_f = 10000.0 ** (-torch.arange(0, d, 2, device="cuda", dtype=torch.float32) / d)
    angles = torch.arange(positions, device="cuda", dtype=torch.float32)[:, None] * inv_f[None, :]
    cos, sin = torch.cos(angles).to(dtype), torch.sin(angles).to(dtype)
    o = rope_attention(q, k, v, cos, sin, causal=causal)
    got = torch.autograd.grad(o, (q, k, v), grad_outputs=do)

    def rotate(x):
        a, b = x.chunk(2, dim=-1)
        c, s = cos[:n].float(), sin[:n].float()
        # The rotated operands are rounded to the storage dtype, as the kernels store them.
        return torch.cat((a * c - b * s, b * c + a * s), dim=-1).to(dtype).float()

    leaves = [t.detach().float().requires_grad_(True) for t in (q, k, v)]
    o_ref = _attention32(rotate(leaves[0]), rotate(leaves[1]), leaves[2], causal)
    refs = torch.autograd.grad(o_ref, leaves, grad_outputs=do.float())
    assert_close(o, o_ref.detach())
    for g, ref in zip(got, refs):
        assert torch.isfinite(g).all()
        assert_relative_frobenius(g, ref, max_relative_error=2e-2)


@pytest.mark.parametrize("case", CASES)
def test_matmul_swiglu(case: int) -> None:
    r = _seeded("matmul_swiglu", case)
    m = int(r.randint(1, 600))
    if case % 2 == 0:  # the fused epilogue kernel (K % 32 == 0, N % 8 == 0)
        n, k = 8 * int(r.randint(1, 100)), 32 * int(r.randint(1, 30))
    else:  # the composition of the GEMM and SwiGLU kernels
        n, k = int(r.randint(1, 500)), int(r.randint(1, 700))
    dtype = DTYPES[(case // 2) % 2]
    torch.manual_seed(case)
    scale = k ** -0.25
    x = (torch.randn(m, k, device="cuda") * scale).to(dtype)
    wg = (torch.randn(k, n, device="cuda") * scale * 2).to(dtype)
    wu = (torch.randn(k, n, device="cuda") * scale).to(dtype)
    xf = x.float()
    assert_close(matmul_swiglu(x, wg, wu), (xf @ wu.float()) * F.silu(xf @ wg.float()))


@pytest.mark.parametrize("case", CASES)
def test_rms_norm_matmul_and_residual_variant(case: int) -> None:
    r = _seeded("rms_norm_matmul", case)
    m = int(r.randint(1, 600))
    # The row-scaled GEMM takes K % 32 == 0 and N % 8 == 0 only (there is no composed path).
    k, n = 32 * int(r.randint(1, 40)), 8 * int(r.randint(1, 100))
    dtype = DTYPES[(case // 2) % 2]
    torch.manual_seed(case)
    x = torch.randn(m, k, device="cuda", dtype=dtype)
    res = torch.randn(m, k, device="cuda", dtype=dtype)
    w_norm = (1 + 0.1 * torch.randn(k, device="cuda")).to(dtype)
    w_proj = (torch.randn(k, n, device="cuda") * k ** -0.5).to(dtype)
    folded = fold_norm_weight(w_norm, w_proj)
    assert torch.equal(folded, (w_norm.float()[:, None] * w_proj.float()).to(dtype))
    out = rms_norm_matmul(x, folded)
    assert_close(out, F.rms_norm(x.float(), (k,), eps=EPS) @ folded.float())
    s, out2 = residual_rms_norm_matmul(x, res, folded)
    assert torch.equal(s, x + res)
    assert_close(out2, F.rms_norm(s.float(), (k,), eps=EPS) @ folded.float())
    with pytest.raises(ValueError, match="K % 32 == 0"):
        rms_norm_matmul(x[:, : k - 1], folded[: k - 1])


@pytest.mark.parametrize("case", CASES)
def test_layer_norm_forward_and_backward(case: int) -> None:
    r = _seeded("layer_norm", case)
    rows = int(r.randint(1, 600))
    cols = int(r.randint(1, 8000))
    dtype = [torch.float16, torch.bfloat16, torch.float32][case % 3]
    torch.manual_seed(case)
    x = (torch.randn(rows, cols, device="cuda") * 2 + 0.5).to(dtype).requires_grad_(True)
    w = (1 + 0.1 * torch.randn(cols, device="cuda")).to(dtype).requires_grad_(True)
    b = (0.1 * torch.randn(cols, device="cuda")).to(dtype).requires_grad_(True)
    dy = torch.randn(rows, cols, device="cuda", dtype=dtype)
    y = layer_norm(x, w, b)
    grads = torch.autograd.grad(y, (x, w, b), grad_outputs=dy)
    leaves = [t.detach().float().requires_grad_(True) for t in (x, w, b)]
    y_ref = F.layer_norm(leaves[0], (cols,), leaves[1], leaves[2], EPS)
    refs = torch.autograd.grad(y_ref, leaves, grad_outputs=dy.float())
    assert_close(y, y_ref)
    assert_close(grads[0], refs[0])
    for g, ref in zip(grads[1:], refs[1:]):
        assert_relative_frobenius(g, ref, max_relative_error=1e-2)


@pytest.mark.parametrize("case", range(8))
def test_activations_forward_and_backward(case: int) -> None:
    r = _seeded("activations", case)
    rows, cols = int(r.randint(1, 300)), int(r.randint(1, 3000))
    dtype = [torch.float16, torch.bfloat16, torch.float32][case % 3]
    fn, ref_fn = [(relu, F.relu), (gelu, F.gelu), (silu, F.silu), (tanh, torch.tanh)][case % 4]
    torch.manual_seed(case)
    x = (torch.randn(rows, cols, device="cuda") * 3).to(dtype).requires_grad_(True)
    dy = torch.randn(rows, cols, device="cuda", dtype=dtype)
    y = fn(x)
    (dx,) = torch.autograd.grad(y, (x,), grad_outputs=dy)
    xf = x.detach().float().requires_grad_(True)
    yf = ref_fn(xf)
    (dxf,) = torch.autograd.grad(yf, (xf,), grad_outputs=dy.float())
    assert_close(y, yf)
    assert_close(dx, dxf)


@pytest.mark.parametrize("case", CASES)
def test_vector_add(case: int) -> None:
    r = _seeded("vector_add", case)
    n = int(r.randint(1, 3_000_000))
    dtype = [torch.float16, torch.bfloat16, torch.float32][case % 3]
    torch.manual_seed(case)
    x = torch.randn(n, device="cuda", dtype=dtype)
    y = torch.randn(n, device="cuda", dtype=dtype)
    assert torch.equal(vector_add(x, y), x + y)
