"""Pins the CPU oracle (oracle/tklab_oracle.c) before it is trusted as the checker.

The reference ships no golden vectors for these kernels (its tests compare
against PyTorch on the GPU), so each oracle function is pinned here against
PyTorch library routines evaluated in float64 on the CPU (softmax, rms_norm,
autograd, SiLU, matmul, scaled_dot_product_attention, logsumexp),
against formulations the oracle does not share (RoPE as a complex
multiplication, attention through the dense softmax matrix) and against closed
forms (constant rows, identity matrices, uniform attention). The storage
roundings are pinned bit-exactly against PyTorch's own casts. Chosen so that a
dropped term, a sign error or a swapped operand fails at least one check.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle



def _rand(*shape, seed=0, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).double()


def _close(a, b, rtol, atol=0.0):
    np.testing.assert_allclose(np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64),
                               rtol=rtol, atol=atol)


# ---------------------------------------------------------------- rounding


@pytest.mark.parametrize(("name", "dtype"), [("bfloat16", torch.bfloat16), ("float16", torch.float16)])
def test_rounding_is_bitwise_torch_cast(name, dtype) -> None:
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 100_000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 5.96e-8, 2.98e-8, -3e-5,
                  3.4e38, np.inf, -np.inf], dtype=np.float32),
        # exact ties at the 16-bit rounding point
        (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0 ** -8) + np.float32(2.0 ** -9)),
    ]).astype(np.float32)
    got = oracle.round_to(x, name)
    want = torch.from_numpy(x).to(dtype).float().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- softmax


def test_softmax_matches_torch_and_closed_forms() -> None:
    x = _rand(64, 1000, seed=2, scale=3.0)
    y = oracle.softmax(x, "float32")
    _close(y, torch.softmax(_t(x), dim=-1).numpy(), rtol=2e-6, atol=1e-9)
    const = np.full((3, 500), 7.25, dtype=np.float32)
    _close(oracle.softmax(const, "float32"), np.full_like(const, 1 / 500), rtol=1e-6)
    # invariant to a per-row shift
    _close(oracle.softmax(x + np.float32(100.0), "float32"), y, rtol=1e-4, atol=1e-7)


def test_softmax_storage_rounding() -> None:
    x = torch.randn(8, 300, dtype=torch.float32).to(torch.bfloat16).float().numpy()
    y = oracle.softmax(x, "bfloat16")
    want = torch.softmax(_t(x), dim=-1).to(torch.bfloat16).double().numpy()
    _close(y, want, rtol=2 ** -7)


# ---------------------------------------------------------------- RMSNorm


def test_rmsnorm_forward_matches_torch() -> None:
    x, w = _rand(50, 777, seed=3), _rand(777, seed=4)
    s, y, rstd = oracle.rmsnorm_fwd(x, w, 1e-5, "float32")
    ref = F.rms_norm(_t(x), (777,), _t(w), 1e-5)
    _close(y, ref.numpy(), rtol=1e-5, atol=1e-6)
    _close(rstd, (1 / torch.sqrt((_t(x) ** 2).mean(-1) + 1e-5)).numpy(), rtol=1e-6)
    assert np.array_equal(s, x)


def test_rmsnorm_constant_row_closed_form() -> None:
    c, eps = 3.0, 1e-6
    x = np.full((2, 64), c, dtype=np.float32)
    w = np.linspace(-1, 1, 64).astype(np.float32)
    _, y, _ = oracle.rmsnorm_fwd(x, w, eps, "float32")
    _close(y, np.tile(w * c / math.sqrt(c * c + eps), (2, 1)), rtol=1e-6)


def test_residual_sum_is_bitwise_torch_add_in_bf16() -> None:
    xb = torch.randn(20, 300, dtype=torch.float32).to(torch.bfloat16)
    rb = torch.randn(20, 300, dtype=torch.float32).to(torch.bfloat16)
    w = torch.ones(300).to(torch.bfloat16)
    s, y, _ = oracle.rmsnorm_fwd(xb.float().numpy(), w.float().numpy(), 1e-6, "bfloat16",
                                 residual=rb.float().numpy())
    assert np.array_equal(s, (xb + rb).float().numpy())
    ref = F.rms_norm((xb + rb).double(), (300,), w.double(), 1e-6).to(torch.bfloat16)
    _close(y, ref.double().numpy(), rtol=2 ** -7)


@pytest.mark.parametrize("with_incoming", [False, True])
def test_rmsnorm_backward_matches_autograd(with_incoming) -> None:
    x, w, dy = _rand(40, 513, seed=5), _rand(513, seed=6), _rand(40, 513, seed=7)
    inc = _rand(40, 513, seed=8) if with_incoming else None
    _, _, rstd = oracle.rmsnorm_fwd(x, w, 1e-5, "float32")
    dx, dw = oracle.rmsnorm_bwd(dy, x, w, rstd, "float32", incoming=inc)
    xt, wt = _t(x).requires_grad_(True), _t(w).requires_grad_(True)
    gx, gw = torch.autograd.grad(F.rms_norm(xt, (513,), wt, 1e-5), (xt, wt), grad_outputs=_t(dy))
    if inc is not None:
        gx = gx + _t(inc)
    _close(dx, gx.numpy(), rtol=1e-4, atol=1e-5)
    _close(dw, gw.numpy(), rtol=1e-5, atol=1e-5)
    # closed form of the weight gradient
    _close(dw, (_t(dy) * _t(x) * _t(rstd)[:, None]).sum(0).numpy(), rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- SwiGLU


def test_swiglu_matches_silu_and_autograd() -> None:
    v, g, dy = _rand(30, 400, seed=9), _rand(30, 400, seed=10, scale=4.0), _rand(30, 400, seed=11)
    _close(oracle.swiglu_fwd(v, g, "float32"), (_t(v) * F.silu(_t(g))).numpy(), rtol=2e-6, atol=1e-7)
    vt, gt = _t(v).requires_grad_(True), _t(g).requires_grad_(True)
    rv, rg = torch.autograd.grad(vt * F.silu(gt), (vt, gt), grad_outputs=_t(dy))
    dv, dg = oracle.swiglu_bwd(dy, v, g, "float32")
    _close(dv, rv.numpy(), rtol=2e-6, atol=1e-7)
    _close(dg, rg.numpy(), rtol=5e-6, atol=1e-6)


def test_swiglu_extreme_gates() -> None:
    g = np.array([[-100, -80, -20, -1, 0, 1, 20, 100]], dtype=np.float32)
    v = np.ones_like(g)
    y = oracle.swiglu_fwd(v, g, "float32")
    dv, dg = oracle.swiglu_bwd(np.ones_like(g), v, g, "float32")
    assert np.isfinite(y).all() and np.isfinite(dv).all() and np.isfinite(dg).all()
    _close(y, F.silu(_t(g)).numpy(), rtol=1e-6, atol=1e-30)


# ---------------------------------------------------------------- RoPE


def _tables(rows, half, seed):
    ang = _rand(rows, half, seed=seed, scale=3.0)
    return ang, np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def test_rope_equals_complex_rotation() -> None:
    rows, half = 33, 64
    x = _rand(rows, 2 * half, seed=12)
    ang, c, s = _tables(rows, half, 13)
    y = oracle.rope_fwd(x, c, s, "float32")
    z = torch.complex(_t(x[:, :half]), _t(x[:, half:])) * torch.complex(_t(c), _t(s))
    _close(y[:, :half], z.real.numpy(), rtol=1e-5, atol=1e-6)
    _close(y[:, half:], z.imag.numpy(), rtol=1e-5, atol=1e-6)
    # rotation by the opposite angle undoes it
    _close(oracle.rope_fwd(y, c, -s, "float32"), x, rtol=1e-4, atol=1e-5)


def test_rope_backward_matches_autograd_of_complex_form() -> None:
    rows, half = 17, 32
    x, dy = _rand(rows, 2 * half, seed=14), _rand(rows, 2 * half, seed=15)
    _, c, s = _tables(rows, half, 16)
    xt, ct, st = (_t(a).requires_grad_(True) for a in (x, c, s))
    z = torch.complex(xt[:, :half], xt[:, half:]) * torch.complex(ct, st)
    out = torch.cat((z.real, z.imag), dim=-1)
    gx, gc, gs = torch.autograd.grad(out, (xt, ct, st), grad_outputs=_t(dy))
    dx, dc, ds = oracle.rope_bwd(dy, x, c, s, "float32")
    _close(dx, gx.numpy(), rtol=1e-5, atol=1e-6)
    _close(dc, gc.numpy(), rtol=1e-5, atol=1e-6)
    _close(ds, gs.numpy(), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- GEMM


def test_gemm_matches_matmul_and_identity() -> None:
    a, b = _rand(37, 91, seed=17), _rand(91, 53, seed=18)
    _close(oracle.gemm(a, b, "float32"), (_t(a) @ _t(b)).numpy(), rtol=1e-6, atol=1e-6)
    assert np.array_equal(oracle.gemm(a, np.eye(91, dtype=np.float32), "float32"), a)
    # non-commuting operands: a transposed-operand mistake would fail
    sq1, sq2 = _rand(16, 16, seed=19), _rand(16, 16, seed=20)
    assert not np.allclose(oracle.gemm(sq1, sq2, "float32"), oracle.gemm(sq2, sq1, "float32"))


def test_gemm_rounds_the_output_once() -> None:
    a = torch.randn(20, 64).to(torch.float16)
    b = torch.randn(64, 30).to(torch.float16)
    got = oracle.gemm(a.float().numpy(), b.float().numpy(), "float16")
    want = (a.double() @ b.double()).to(torch.float16).double().numpy()
    _close(got, want, rtol=2 ** -10)


# ---------------------------------------------------------------- attention


@pytest.mark.parametrize("causal", [False, True])
def test_attention_forward_matches_sdpa_and_lse(causal) -> None:
    q, k, v = (_rand(2, 3, 70, 32, seed=s) for s in (21, 22, 23))
    o, lse = oracle.attn_fwd(q, k, v, 32 ** -0.5, causal, "float32")
    ref = F.scaled_dot_product_attention(_t(q), _t(k), _t(v), is_causal=causal)
    _close(o, ref.numpy(), rtol=1e-5, atol=1e-6)
    scores = _t(q) @ _t(k).transpose(-2, -1) * 32 ** -0.5
    if causal:
        scores = scores.masked_fill(torch.triu(torch.ones(70, 70, dtype=torch.bool), 1), -math.inf)
    _close(lse, (torch.logsumexp(scores, -1) * math.log2(math.e)).numpy(), rtol=1e-6, atol=1e-6)


def test_attention_uniform_keys_give_value_means() -> None:
    q, v = _rand(1, 1, 40, 16, seed=24), _rand(1, 1, 40, 16, seed=25)
    k = np.zeros_like(q)
    o, lse = oracle.attn_fwd(q, k, v, 0.25, True, "float32")
    prefix = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, 41)[:, None]
    _close(o, prefix, rtol=1e-5, atol=1e-6)
    _close(lse[0, 0], np.log2(np.arange(1, 41)), rtol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_backward_matches_autograd(causal) -> None:
    q, k, v, do = (_rand(1, 2, 45, 16, seed=s) for s in (26, 27, 28, 29))
    scale = 16 ** -0.5
    o, lse = oracle.attn_fwd(q, k, v, scale, causal, "float32")
    dq, dk, dv = oracle.attn_bwd(q, k, v, o, do, lse, scale, causal, "float32")
    qt, kt, vt = (_t(a).requires_grad_(True) for a in (q, k, v))
    s = qt @ kt.transpose(-2, -1) * scale
    if causal:
        s = s.masked_fill(torch.triu(torch.ones(45, 45, dtype=torch.bool), 1), -math.inf)
    out = torch.softmax(s, -1) @ vt
    refs = torch.autograd.grad(out, (qt, kt, vt), grad_outputs=_t(do))
    for got, want in zip((dq, dk, dv), refs):
        _close(got, want.numpy(), rtol=1e-4, atol=1e-5)


def test_attention_bf16_operand_rounding_stays_within_the_dtype_bound() -> None:
    q, k, v = (torch.randn(1, 1, 64, 32).to(torch.bfloat16).float().numpy() for _ in range(3))
    o, _ = oracle.attn_fwd(q, k, v, 32 ** -0.5, False, "bfloat16")
    ref = F.scaled_dot_product_attention(_t(q), _t(k), _t(v))
    assert np.max(np.abs(o - ref.numpy())) < 2e-2


# ---------------------------------------------------------------- GQA decode


def test_gqa_decode_is_the_last_row_of_causal_attention() -> None:
    """G = 1, full length: one decode row is row L-1 of causal attention (same loops)."""
    q_full, k, v = (_rand(2, 3, 37, 32, seed=s) for s in (41, 42, 43))
    for dt in ("float32", "bfloat16"):
        o_full, lse_full = oracle.attn_fwd(q_full, k, v, 32 ** -0.5, True, dt)
        o, lse = oracle.gqa_decode(q_full[:, :, -1], k, v, 32 ** -0.5, dt)
        np.testing.assert_array_equal(o, o_full[:, :, -1])
        np.testing.assert_array_equal(lse, lse_full[:, :, -1])


def test_gqa_decode_equals_repeated_kv_heads_and_truncated_caches() -> None:
    q = _rand(3, 8, 64, seed=44)
    k, v = _rand(3, 2, 50, 64, seed=45), _rand(3, 2, 50, 64, seed=46)
    lens = np.array([50, 17, 1], dtype=np.int32)
    o, lse = oracle.gqa_decode(q, k, v, 0.125, "bfloat16", lens)
    # kv_head(h) = h // 4: repeating each KV head 4 times makes it plain multi-head.
    o_rep, lse_rep = oracle.gqa_decode(
        q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), 0.125, "bfloat16", lens
    )
    np.testing.assert_array_equal(o, o_rep)
    np.testing.assert_array_equal(lse, lse_rep)
    for b, n in enumerate(lens):
        o_b, lse_b = oracle.gqa_decode(
            q[b : b + 1], np.ascontiguousarray(k[b : b + 1, :, :n]),
            np.ascontiguousarray(v[b : b + 1, :, :n]), 0.125, "bfloat16",
        )
        np.testing.assert_array_equal(o[b], o_b[0])
        np.testing.assert_array_equal(lse[b], lse_b[0])
    o0, lse0 = oracle.gqa_decode(q, k, v, 0.125, "float32", np.array([0, 5, 99], dtype=np.int32))
    assert np.all(o0[0] == 0) and np.all(np.isneginf(lse0[0]))
    np.testing.assert_array_equal(
        o0[2], oracle.gqa_decode(q, k, v, 0.125, "float32")[0][2]
    )  # lengths above L read the whole cache


def test_gqa_decode_matches_sdpa_with_grouped_heads() -> None:
    q = _rand(2, 8, 1, 32, seed=47)
    k, v = _rand(2, 2, 40, 32, seed=48), _rand(2, 2, 40, 32, seed=49)
    o, lse = oracle.gqa_decode(q[:, :, 0], k, v, 32 ** -0.5, "float32")
    ref = F.scaled_dot_product_attention(_t(q), _t(k), _t(v), enable_gqa=True)
    _close(o, ref[:, :, 0].numpy(), rtol=1e-5, atol=1e-6)
    scores = _t(q) @ _t(np.repeat(k, 4, axis=1)).transpose(-2, -1) * 32 ** -0.5
    _close(lse, (torch.logsumexp(scores, -1)[:, :, 0] * math.log2(math.e)).numpy(), rtol=1e-6,
           atol=1e-6)
