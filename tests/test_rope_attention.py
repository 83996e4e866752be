"""GPU parity of RoPE'd attention (tk_attn_fwd_rope, tk_rope_positions).

rope_attention(q, k, v, cos, sin) must be, bit for bit, the composition
rope(q), rope(k) (the reference-contract RoPE with per-row tables expanded from the
position tables) followed by grouped_query_attention, forward and backward: Q is
rotated in the attention prologue with the RoPE kernel's arithmetic, and the backward
runs the same kernels on the same rotated tensors. The oracle pins one case end to end.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits_equal, dev, host, name
from oracle import oracle
from tklab import _hip
from tklab.harness.tolerances import assert_close
from tklab.kernels.flash_attention import grouped_query_attention, rope_attention
from tklab.kernels.rope import rope

pytestmark = pytest.mark.gpu


def _tables(positions, half, dtype):
    inv = 10000.0 ** (-torch.arange(half, dtype=torch.float32) / half)
    ang = torch.arange(positions, dtype=torch.float32)[:, None] * inv[None]
    return ang.cos().to(dtype).cuda(), ang.sin().to(dtype).cuda()


def _inputs(b, h, hkv, n, d, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(b, h, n, d, device="cuda", dtype=dtype, generator=g)
    k = torch.randn(b, hkv, n, d, device="cuda", dtype=dtype, generator=g)
    v = torch.randn(b, hkv, n, d, device="cuda", dtype=dtype, generator=g)
    do = torch.randn(b, h, n, d, device="cuda", dtype=dtype, generator=g)
    return q, k, v, do


def _rope_rows(x, cos, sin):
    """The reference-contract RoPE on (b, h, n, d) with position tables expanded per row."""
    b, h, n, d = x.shape
    c = cos[:n].repeat(b * h, 1).contiguous()
    s = sin[:n].repeat(b * h, 1).contiguous()
    return rope(x.reshape(b * h * n, d), c, s).reshape(b, h, n, d)


def _grads(fn, tensors, do):
    leaves = [t.detach().clone().requires_grad_(True) for t in tensors]
    out = fn(*leaves)
    out.backward(do)
    return [out.detach()] + [t.grad for t in leaves]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d,h,hkv", [(128, 4, 2), (64, 4, 4), (128, 8, 1)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_forward_and_backward_are_bitwise_the_composition(causal, d, h, hkv, dtype) -> None:
    n = 200  # ragged against the 256-query and 64-key blocks; tables have spare rows
    q, k, v, do = _inputs(2, h, hkv, n, d, dtype, seed=d + h + causal)
    cos, sin = _tables(n + 7, d // 2, dtype)
    got = _grads(lambda a, b, c: rope_attention(a, b, c, cos, sin, causal=causal), (q, k, v), do)
    want = _grads(
        lambda a, b, c: grouped_query_attention(
            _rope_rows(a, cos, sin), _rope_rows(b, cos, sin), c, causal=causal
        ),
        (q, k, v),
        do,
    )
    for g_t, w_t in zip(got, want):
        assert bits_equal(g_t, w_t)


def test_positions_rope_is_the_per_row_rope() -> None:
    x = torch.randn(3, 5, 77, 128, device="cuda", dtype=torch.bfloat16)
    cos, sin = _tables(90, 64, torch.bfloat16)
    for inverse in (False, True):
        out = torch.empty_like(x)
        _hip.call("tk_rope_positions", _hip.dtype_code(x.dtype), x.data_ptr(), cos.data_ptr(),
                  sin.data_ptr(), out.data_ptr(), 3 * 5 * 77, 77, 64, 128, cos.stride(0), 128,
                  int(inverse), _hip.stream_of(x))
        c = cos[:77].repeat(15, 1).contiguous()
        s = sin[:77].repeat(15, 1).contiguous()
        flat = x.reshape(-1, 128)
        if inverse:  # RoPE's input gradient is RoPE with -sin
            leaf = flat.clone().requires_grad_(True)
            rope(leaf, c, s).backward(flat)
            want = leaf.grad
        else:
            want = rope(flat, c, s)
        assert bits_equal(out.reshape(-1, 128), want)


def test_identity_tables_give_plain_attention() -> None:
    q, k, v, _ = _inputs(1, 8, 2, 300, 128, torch.bfloat16, seed=11)
    ones = torch.ones(300, 64, device="cuda", dtype=torch.bfloat16)
    zeros = torch.zeros_like(ones)
    with torch.no_grad():
        got = rope_attention(q, k, v, ones, zeros, causal=True)
        want = grouped_query_attention(q, k, v, causal=True)
    assert bits_equal(got, want)


def test_matches_the_oracle() -> None:
    q, k, v, _ = _inputs(1, 4, 2, 150, 64, torch.float16, seed=12)
    cos, sin = _tables(150, 32, torch.float16)
    with torch.no_grad():
        out = rope_attention(q, k, v, cos, sin, causal=True)

    def rot(x):  # float32 rotate-half, products rounded separately, then to float16
        x = host(x).astype(np.float32)
        c, s = host(cos).astype(np.float32), host(sin).astype(np.float32)
        x1, x2 = x[..., :32], x[..., 32:]
        y = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
        return y.astype(np.float16)

    qr = rot(q)
    kr = np.repeat(rot(k), 2, axis=1)
    vr = np.repeat(host(v), 2, axis=1)
    o_ref, _ = oracle.attn_fwd(qr, kr, vr, 64 ** -0.5, True, name(q.dtype))
    assert_close(out, dev(o_ref, out))


def test_contract() -> None:
    q, k, v, _ = _inputs(1, 4, 2, 64, 64, torch.bfloat16, seed=13)
    cos, sin = _tables(64, 32, torch.bfloat16)
    with pytest.raises(ValueError, match="row per sequence position"):
        rope_attention(q, k, v, cos[:63], sin[:63], causal=True)
    with pytest.raises(ValueError, match=r"\(positions, head_dim // 2\)"):
        rope_attention(q, k, v, cos[:, :16], sin[:, :16], causal=True)
    with pytest.raises(ValueError, match="dtype and device"):
        rope_attention(q, k, v, cos.half(), sin.half(), causal=True)
    with pytest.raises(ValueError, match="multiple of the K/V heads"):
        rope_attention(q[:, :3], k, v, cos, sin, causal=True)
