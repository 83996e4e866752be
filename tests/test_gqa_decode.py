"""GPU parity of tk_gqa_decode against the CPU oracle and PyTorch SDPA."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from _helpers import dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close
from tklab.kernels.gqa_decode import gqa_decode

pytestmark = pytest.mark.gpu


def _case(batch, q_heads, kv_heads, length, d, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(batch, q_heads, d, device="cuda", dtype=dtype, generator=g)
    k = torch.randn(batch, kv_heads, length, d, device="cuda", dtype=dtype, generator=g)
    v = torch.randn(batch, kv_heads, length, d, device="cuda", dtype=dtype, generator=g)
    return q, k, v


def _check(q, k, v, lens=None):
    d = q.shape[-1]
    o, lse = gqa_decode(q, k, v, lens, return_lse=True)
    o_ref, lse_ref = oracle.gqa_decode(
        host(q), host(k.contiguous()), host(v.contiguous()), d ** -0.5, name(q.dtype),
        None if lens is None else lens.cpu().numpy(),
    )
    assert_close(o, dev(o_ref, o))
    # Float32 statistics: a relative error of 1e-5 in the base-2 LSE.
    torch.testing.assert_close(lse, dev(lse_ref, lse), rtol=1e-5, atol=1e-5)
    return o, lse


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_groups_head_dims_and_dtypes(dtype, d, group) -> None:
    q, k, v = _case(2, 4 * group, 4, 777, d, dtype, seed=group * 10 + d)
    _check(q, k, v)


@pytest.mark.parametrize("length", [1, 31, 32, 33, 64, 65, 1000, 4096])
def test_cache_lengths_and_block_edges(length) -> None:
    q, k, v = _case(3, 32, 8, length, 128, torch.bfloat16, seed=length)
    _check(q, k, v)


def test_variable_lengths_including_empty_and_clamped() -> None:
    q, k, v = _case(5, 8, 2, 3000, 128, torch.bfloat16, seed=5)
    lens = torch.tensor([3000, 1, 0, 1537, 9999], device="cuda", dtype=torch.int32)
    o, lse = _check(q, k, v, lens)
    assert torch.all(o[2] == 0) and torch.all(torch.isneginf(lse[2]))


def test_sequence_major_cache_layout() -> None:
    """A [batch, max_len, kv_heads, d] cache read through head-major strides."""
    g = torch.Generator(device="cuda").manual_seed(6)
    q = torch.randn(2, 16, 128, device="cuda", dtype=torch.bfloat16, generator=g)
    k = torch.randn(2, 500, 4, 128, device="cuda", dtype=torch.bfloat16, generator=g)
    v = torch.randn(2, 500, 4, 128, device="cuda", dtype=torch.bfloat16, generator=g)
    _check(q, k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3))


def test_matches_sdpa_with_grouped_heads() -> None:
    q, k, v = _case(4, 32, 8, 2048, 128, torch.bfloat16, seed=7)
    o = gqa_decode(q, k, v)
    ref = F.scaled_dot_product_attention(
        q.float()[:, :, None], k.float(), v.float(), enable_gqa=True
    )[:, :, 0]
    assert_close(o, ref.to(o.dtype))


def test_equals_last_row_of_causal_attention_forward() -> None:
    """G = 1: the decode row is row L-1 of the library's causal attention forward."""
    from tklab.kernels.flash_attention import _launch_forward

    g = torch.Generator(device="cuda").manual_seed(8)
    q, k, v = (torch.randn(1, 8, 256, 128, device="cuda", dtype=torch.bfloat16, generator=g)
               for _ in range(3))
    o = torch.empty_like(q)
    lse = torch.empty(1, 8, 256, device="cuda")
    _launch_forward(q, k, v, o, lse, causal=True, store_lse=True)
    od, lsed = gqa_decode(q[:, :, -1].contiguous(), k, v, return_lse=True)
    assert_close(od, o[:, :, -1])
    torch.testing.assert_close(lsed, lse[:, :, -1], rtol=1e-5, atol=1e-5)


def test_results_are_bitwise_reproducible() -> None:
    q, k, v = _case(2, 32, 8, 5000, 128, torch.bfloat16, seed=9)
    a = gqa_decode(q, k, v)
    b = gqa_decode(q, k, v)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("group", [1, 4, 8])
def test_one_split_writes_the_output_directly(dtype, d, group, monkeypatch) -> None:
    """With one split per (batch, KV head) the split wave normalizes and writes O and the LSE
    (no combine pass); empty and clamped lengths write O = 0, LSE = -inf."""
    import tklab.kernels.gqa_decode as gd

    monkeypatch.setattr(gd, "split_length", lambda b, h, n: max(64, -(-n // 64) * 64))
    q, k, v = _case(4, 2 * group, 2, 1500, d, dtype, seed=30 + group + d)
    _check(q, k, v)
    lens = torch.tensor([1500, 0, 1, 777], device="cuda", dtype=torch.int32)
    o, lse = _check(q, k, v, lens)
    assert torch.all(o[1] == 0) and torch.all(torch.isneginf(lse[1]))

