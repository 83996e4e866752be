"""GPU parity of the flash-attention forward (tk_attn_fwd).

Reference checks (tests/test_flash_attention.py of the reference): SDPA
agreement within relative Frobenius 2e-2 for (1, 16, N, 64) float16 at
N = 128 and 1000, seeds 23 + N + causal; the saved statistic equals
logsumexp(scores) * log2(e) within 1e-3, seeds 91 + causal. References are
evaluated on float32 upcasts. This build adds the CPU oracle across dtypes and
head dims, and a per-head float32 check at the benchmark shape.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from _helpers import dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.flash_attention import _launch_forward, attention_causal, attention_noncausal

pytestmark = pytest.mark.gpu

KERNELS = [(False, attention_noncausal), (True, attention_causal)]


def _sdpa32(q, k, v, causal):
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=causal)


def _scores32(q, k, causal):
    s = torch.matmul(q.float(), k.float().transpose(-2, -1).contiguous()) / math.sqrt(q.shape[-1])
    if causal:
        n = q.shape[-2]
        mask = torch.triu(torch.ones(n, n, dtype=torch.bool, device=q.device), diagonal=1)
        s = s.masked_fill(mask, -torch.inf)
    return s


@pytest.mark.parametrize(("causal", "kernel"), KERNELS)
@pytest.mark.parametrize("n", [128, 1000])
def test_matches_sdpa(causal, kernel, n) -> None:
    torch.manual_seed(23 + n + int(causal))
    q, k, v = (torch.randn(1, 16, n, 64, device="cuda", dtype=torch.float16) for _ in range(3))
    out = kernel(q, k, v)
    assert torch.isfinite(out).all()
    assert_relative_frobenius(out, _sdpa32(q, k, v, causal), max_relative_error=2e-2)


@pytest.mark.parametrize("causal", [False, True])
def test_saved_statistic_is_base2_logsumexp(causal) -> None:
    torch.manual_seed(91 + int(causal))
    shape = (1, 2, 129, 64)
    q, k, v = (torch.randn(shape, device="cuda", dtype=torch.float16) for _ in range(3))
    out = torch.empty_like(q)
    lse = torch.empty(shape[:-1], device="cuda", dtype=torch.float32)
    _launch_forward(q, k, v, out, lse, causal=causal, store_lse=True)
    expected = torch.logsumexp(_scores32(q, k, causal), dim=-1) * math.log2(math.e)
    assert torch.isfinite(lse).all()
    assert_relative_frobenius(lse, expected, max_relative_error=1e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [1, 63, 129, 300, 513])
def test_matches_the_oracle(dtype, d, causal, n) -> None:
    torch.manual_seed(n + d + int(causal))
    shape = (2, 2, n, d)
    q, k, v = (torch.randn(shape, device="cuda", dtype=dtype) for _ in range(3))
    out = torch.empty_like(q)
    lse = torch.empty(shape[:-1], device="cuda", dtype=torch.float32)
    _launch_forward(q, k, v, out, lse, causal=causal, store_lse=True)
    o_ref, lse_ref = oracle.attn_fwd(host(q), host(k), host(v), d ** -0.5, causal, name(dtype))
    assert_close(out, dev(o_ref, out))
    assert_relative_frobenius(out, dev(o_ref, out), max_relative_error=1e-2)
    # FP32 statistic: 1e-5 relative.
    torch.testing.assert_close(lse, dev(lse_ref, lse), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("kind", ["ramp", "large"])
def test_running_maximum_moves_often(dtype, d, causal, kind) -> None:
    """Scores that grow along the keys (each 64-key block's maximum exceeds the previous
    block's by far more than 2^8 in base 2) and large random logits: the kernel's reference
    maximum moves in most blocks, and the result still matches the oracle."""
    torch.manual_seed(17 + d + int(causal))
    n = 300
    shape = (1, 2, n, d)
    if kind == "ramp":
        q = 1 + 0.1 * torch.randn(shape, device="cuda")
        ramp = (0.1 * torch.arange(n, device="cuda", dtype=torch.float32))[:, None]
        k = ramp + 0.1 * torch.randn(shape, device="cuda")
    else:
        q = 6 * torch.randn(shape, device="cuda")
        k = torch.randn(shape, device="cuda")
    q, k = q.to(dtype), k.to(dtype)
    v = torch.randn(shape, device="cuda", dtype=dtype)
    out = torch.empty_like(q)
    lse = torch.empty(shape[:-1], device="cuda", dtype=torch.float32)
    _launch_forward(q, k, v, out, lse, causal=causal, store_lse=True)
    o_ref, lse_ref = oracle.attn_fwd(host(q), host(k), host(v), d ** -0.5, causal, name(dtype))
    assert torch.isfinite(out).all()
    assert_close(out, dev(o_ref, out))
    torch.testing.assert_close(lse, dev(lse_ref, lse), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n", [513, 768])
def test_paired_causal_blocks_on_the_xcd_path(n) -> None:
    """Causal head_dim 128 deals query blocks i and QB-1-i to one workgroup: batch x heads
    a multiple of 8 (each XCD takes its eighth of the heads) and an odd block count (the
    middle block has no partner), against the oracle."""
    torch.manual_seed(n + 1)
    shape = (2, 4, n, 128)
    q, k, v = (torch.randn(shape, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    out = torch.empty_like(q)
    lse = torch.empty(shape[:-1], device="cuda", dtype=torch.float32)
    _launch_forward(q, k, v, out, lse, causal=True, store_lse=True)
    o_ref, lse_ref = oracle.attn_fwd(host(q), host(k), host(v), 128 ** -0.5, True, "bfloat16")
    assert_close(out, dev(o_ref, out))
    assert_relative_frobenius(out, dev(o_ref, out), max_relative_error=1e-2)
    torch.testing.assert_close(lse, dev(lse_ref, lse), rtol=1e-5, atol=1e-5)


def test_inference_and_training_forward_agree_bitwise() -> None:
    torch.manual_seed(5)
    q, k, v = (torch.randn(1, 4, 700, 128, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    with torch.no_grad():
        a = attention_causal(q, k, v)
    q.requires_grad_(True)
    b = attention_causal(q, k, v)
    assert torch.equal(a, b.detach())


def test_single_key_and_constant_keys_closed_forms() -> None:
    torch.manual_seed(6)
    q = torch.randn(1, 2, 300, 64, device="cuda", dtype=torch.float16)
    v = torch.randn_like(q)
    k = torch.zeros_like(q)  # equal scores: uniform weights
    out = attention_causal(q, k, v)
    prefix_mean = torch.cumsum(v.float(), dim=2) / torch.arange(1, 301, device="cuda")[:, None]
    assert_relative_frobenius(out, prefix_mean, max_relative_error=2e-3)
    torch.testing.assert_close(out[:, :, 0], v[:, :, 0], rtol=0, atol=0)
    out_nc = attention_noncausal(q, k, v)
    torch.testing.assert_close(
        out_nc.float(), v.float().mean(dim=2, keepdim=True).expand_as(out_nc), rtol=2e-3, atol=2e-3
    )


@pytest.mark.parametrize(
    ("causal", "n", "d"), [(True, 8192, 128), (False, 4096, 128), (True, 8192, 64), (False, 4096, 64)]
)
def test_config_shapes_per_head(causal, n, d) -> None:
    """benchmark config 5 shapes (B4 H32 bf16): every head finite; eight heads, two in each
    batch, checked against float32 torch math (output and base-2 LSE)."""
    torch.manual_seed(0)
    shape = (4, 32, n, d)
    q, k, v = (torch.randn(shape, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    out = torch.empty_like(q)
    lse = torch.empty(shape[:-1], device="cuda", dtype=torch.float32)
    _launch_forward(q, k, v, out, lse, causal=causal, store_lse=True)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    for b, h in ((0, 0), (0, 19), (1, 6), (1, 31), (2, 12), (2, 25), (3, 3), (3, 31)):
        print(f"config-5 forward head ({b}, {h})", flush=True)
        s = _scores32(q[b, h], k[b, h], causal)
        ref = torch.softmax(s, dim=-1) @ v[b, h].float()
        assert_relative_frobenius(out[b, h], ref, max_relative_error=1e-2)
        assert_relative_frobenius(
            lse[b, h], torch.logsumexp(s, dim=-1) * math.log2(math.e), max_relative_error=1e-5
        )


def _abi_forward(q, k, v, causal):
    """tk_attn_fwd through the C ABI with the tensors' own (possibly strided) layouts."""
    from tklab import _hip

    batch, heads, n_ctx, head_dim = q.shape
    out = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    lse = torch.empty(q.shape[:-1], device=q.device, dtype=torch.float32)
    strides = lambda t: _hip.int64_array(list(t.stride()[:3]))  # noqa: E731
    _hip.call("tk_attn_fwd", _hip.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), v.data_ptr(),
              out.data_ptr(), lse.data_ptr(), batch, heads, n_ctx, head_dim, strides(q),
              strides(k), strides(v), strides(out), 1.0 / math.sqrt(head_dim), int(causal),
              _hip.stream_of(q))
    return out, lse


@pytest.mark.parametrize("causal", [False, True])
def test_sequence_major_layout_through_the_abi(causal) -> None:
    """[batch, seq, heads, dim] storage viewed as (B, H, N, D): sequence stride H * D."""
    torch.manual_seed(11 + int(causal))
    shape = (2, 333, 3, 128)
    q, k, v = (torch.randn(shape, device="cuda", dtype=torch.bfloat16).transpose(1, 2)
               for _ in range(3))
    out, lse = _abi_forward(q, k, v, causal)
    o_ref, lse_ref = oracle.attn_fwd(host(q.contiguous()), host(k.contiguous()),
                                     host(v.contiguous()), 128 ** -0.5, causal, "bfloat16")
    assert_close(out, dev(o_ref, out))
    torch.testing.assert_close(lse, dev(lse_ref, lse), rtol=1e-5, atol=1e-5)


def test_head_rows_spanning_two_gib_take_the_register_staged_kernel() -> None:
    """K rows 2^20 elements apart (2.2 GiB per head) exceed 32-bit buffer offsets."""
    torch.manual_seed(12)
    n, d, stride = 1100, 64, 1 << 20
    q, v = (torch.randn(1, 1, n, d, device="cuda", dtype=torch.float16) for _ in range(2))
    backing = torch.empty(n, stride, device="cuda", dtype=torch.float16)
    backing[:, :d] = torch.randn(n, d, device="cuda", dtype=torch.float16)
    k = backing[:, :d].unsqueeze(0).unsqueeze(0)  # (1, 1, n, d), sequence stride 2^20
    out, lse = _abi_forward(q, k, v, True)
    o_ref, lse_ref = oracle.attn_fwd(host(q), host(k.contiguous()), host(v), d ** -0.5, True,
                                     "float16")
    del backing
    assert_close(out, dev(o_ref, out))
    torch.testing.assert_close(lse, dev(lse_ref, lse), rtol=1e-5, atol=1e-5)
