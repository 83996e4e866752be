"""GPU parity of variable-length attention (tk_attn_*_varlen).

Each packed sequence must get exactly what the library's fixed-length kernels give it
alone (the same tiles in the same order: bitwise equal outputs and gradients), and
match the CPU oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _helpers import bits_equal, dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.flash_attention import grouped_query_attention, varlen_attention

pytestmark = pytest.mark.gpu


def _packed(lengths, heads, kv_heads, d, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    total = sum(lengths)
    q = torch.randn(total, heads, d, device="cuda", dtype=dtype, generator=g)
    k = torch.randn(total, kv_heads, d, device="cuda", dtype=dtype, generator=g)
    v = torch.randn(total, kv_heads, d, device="cuda", dtype=dtype, generator=g)
    do = torch.randn(total, heads, d, device="cuda", dtype=dtype, generator=g)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), device="cuda", dtype=torch.int32)
    return q, k, v, do, cu


def _run(fn, tensors, do):
    leaves = [t.detach().clone().requires_grad_(True) for t in tensors]
    out = fn(*leaves)
    out.backward(do)
    return [out.detach()] + [t.grad for t in leaves]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d,heads,kv_heads", [(128, 4, 4), (64, 8, 2)])
def test_each_sequence_matches_its_fixed_length_run_bitwise(causal, d, heads, kv_heads) -> None:
    lengths = [1, 200, 64, 517, 0, 129]
    q, k, v, do, cu = _packed(lengths, heads, kv_heads, d, torch.bfloat16, seed=d + causal)
    got = _run(lambda a, b, c: varlen_attention(a, b, c, cu, max(lengths), causal=causal),
               (q, k, v), do)
    for i, n in enumerate(lengths):
        if n == 0:
            continue
        s0, s1 = int(cu[i]), int(cu[i + 1])
        seq = [t[s0:s1].transpose(0, 1).unsqueeze(0).contiguous() for t in (q, k, v, do)]
        want = _run(lambda a, b, c: grouped_query_attention(a, b, c, causal=causal),
                    seq[:3], seq[3])
        for g_t, w_t in zip(got, want):
            assert bits_equal(g_t[s0:s1], w_t[0].transpose(0, 1))


def test_matches_the_oracle() -> None:
    lengths = [300, 77]
    q, k, v, do, cu = _packed(lengths, 4, 2, 64, torch.float16, seed=3)
    out, dq, dk, dv = _run(lambda a, b, c: varlen_attention(a, b, c, cu, 300, causal=True),
                           (q, k, v), do)
    for i, n in enumerate(lengths):
        s0, s1 = int(cu[i]), int(cu[i + 1])
        qh = host(q[s0:s1]).transpose(1, 0, 2)[None]
        kh = np.repeat(host(k[s0:s1]).transpose(1, 0, 2)[None], 2, axis=1)
        vh = np.repeat(host(v[s0:s1]).transpose(1, 0, 2)[None], 2, axis=1)
        doh = host(do[s0:s1]).transpose(1, 0, 2)[None]
        o_ref, lse_ref = oracle.attn_fwd(qh, kh, vh, 64 ** -0.5, True, name(q.dtype))
        assert_close(out[s0:s1], dev(o_ref[0].transpose(1, 0, 2), out))
        dq_r, dk_r, dv_r = oracle.attn_bwd(qh, kh, vh, o_ref, doh, lse_ref, 64 ** -0.5, True,
                                           name(q.dtype))
        dk_g = dk_r[0].reshape(2, 2, n, 64).sum(1).transpose(1, 0, 2)
        dv_g = dv_r[0].reshape(2, 2, n, 64).sum(1).transpose(1, 0, 2)
        assert_relative_frobenius(dq[s0:s1], dev(dq_r[0].transpose(1, 0, 2), dq),
                                  max_relative_error=1e-2)
        assert_relative_frobenius(dk[s0:s1], dev(dk_g, dk), max_relative_error=1e-2)
        assert_relative_frobenius(dv[s0:s1], dev(dv_g, dv), max_relative_error=1e-2)


def test_malformed_offsets_stay_inside_the_tensors() -> None:
    """Offsets past total or decreasing are rejected on the host by default; without the
    host check the kernels clamp them: no fault, finite output."""
    q, k, v, _, _ = _packed([100, 100], 2, 2, 64, torch.bfloat16, seed=4)
    cu = torch.tensor([0, 150, 90, 10_000], device="cuda", dtype=torch.int32)
    with pytest.raises(ValueError):
        varlen_attention(q, k, v, cu, 150, causal=True)
    with torch.no_grad():
        out = varlen_attention(q, k, v, cu, 150, causal=True, check_offsets=False)
    torch.cuda.synchronize()
    assert torch.isfinite(out[:150].float()).all()


def test_contract() -> None:
    q, k, v, _, cu = _packed([10, 20], 4, 2, 64, torch.bfloat16, seed=5)
    with pytest.raises(ValueError, match="int32 vector"):
        varlen_attention(q, k, v, cu.long(), 20, causal=True)
    with pytest.raises(ValueError, match="max_seqlen"):
        varlen_attention(q, k, v, cu, 0, causal=True)
    with pytest.raises(ValueError, match="total, heads, dim"):
        varlen_attention(q[None], k, v, cu, 20, causal=True)


@pytest.mark.parametrize("check_offsets", [True, False])
def test_padded_packing_zeroes_rows_outside_every_sequence(check_offsets) -> None:
    """Tokens before cu[0] and after cu[-1] belong to no sequence: zero output and gradients;
    the sequences themselves match the unpadded packing bitwise."""
    lengths = [130, 64, 7]
    lead, tail = 5, 40
    q, k, v, do, cu = _packed(lengths, 4, 2, 128, torch.bfloat16, seed=71)
    total = q.shape[0]
    pad = lambda t: torch.cat([torch.randn(lead, *t.shape[1:], device="cuda", dtype=t.dtype), t,  # noqa: E731
                               torch.randn(tail, *t.shape[1:], device="cuda", dtype=t.dtype)])
    qp, kp, vp, dop = (pad(t) for t in (q, k, v, do))
    cup = cu + lead
    got = _run(lambda a, b, c: varlen_attention(a, b, c, cup, max(lengths), causal=True,
                                                check_offsets=check_offsets), (qp, kp, vp), dop)
    want = _run(lambda a, b, c: varlen_attention(a, b, c, cu, max(lengths), causal=True),
                (q, k, v), do)
    for g_t, w_t in zip(got, want):
        assert bits_equal(g_t[lead:lead + total], w_t)
        assert not g_t[:lead].any() and not g_t[lead + total:].any()


def test_invalid_offsets_are_rejected_on_the_host() -> None:
    q, k, v, _, cu = _packed([10, 20], 2, 2, 64, torch.float16, seed=72)
    bad = [
        (torch.tensor([0, 20, 10], device="cuda", dtype=torch.int32), 20, "non-decreasing"),
        (torch.tensor([0, 10, 31], device="cuda", dtype=torch.int32), 21, r"\[0, total\]"),
        (torch.tensor([-1, 10, 30], device="cuda", dtype=torch.int32), 20, r"\[0, total\]"),
        (cu, 19, "longest sequence"),
    ]
    for offsets, max_len, match in bad:
        with pytest.raises(ValueError, match=match):
            varlen_attention(q, k, v, offsets, max_len, causal=False)
