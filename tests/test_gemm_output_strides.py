"""GPU checks of the GEMM kernels' output paths through the C ABI: tk_gemm, tk_gemm_rowscale
and tk_gemm_swiglu write C (or Y) by three routes, chosen from the output's layout:

- rows 16-byte aligned (unit column stride, row stride a multiple of 8 elements, base
  16-byte aligned): the tile is staged in LDS and written back as whole rows;
- rows 8-byte aligned: each lane stores its four columns as one 8-byte write;
- anything else (odd row stride, column stride above 1): element by element.

Each strided output must equal, bit for bit, the same entry point's contiguous result, and
no element outside the output view may change.
"""

from __future__ import annotations

import pytest
import torch

from _helpers import bits_equal
from tklab import _hip

pytestmark = pytest.mark.gpu

M, N, K = 300, 264, 128  # M and N end inside a block tile; the DMA kernel applies
_INT = {torch.float16: torch.int16, torch.bfloat16: torch.int16}

# (row stride - N, column stride, base offset in elements): staged, 8-byte, element paths.
LAYOUTS = [(8, 1, 0), (24, 1, 8), (4, 1, 0), (8, 1, 4), (1, 1, 0), (0, 2, 0), (3, 3, 1)]


def _operands(dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    sc = K ** -0.25
    a = (torch.randn(M, K, device="cuda", generator=g) * sc).to(dtype)
    b = (torch.randn(K, N, device="cuda", generator=g) * sc).to(dtype)
    b2 = (torch.randn(K, N, device="cuda", generator=g) * sc).to(dtype)
    scale = (1 + 0.25 * torch.rand(M, device="cuda", generator=g)).float()
    return a, b, b2, scale


def _call(entry, dtype, a, b, b2, scale, out_ptr, stride_m, stride_n):
    code = _hip.dtype_code(dtype)
    stream = _hip.stream_of(a)
    if entry == "tk_gemm":
        _hip.call("tk_gemm", code, a.data_ptr(), b.data_ptr(), out_ptr, M, N, K, a.stride(0),
                  a.stride(1), b.stride(0), b.stride(1), stride_m, stride_n, 0, stream)
    elif entry == "tk_gemm_rowscale":
        _hip.call("tk_gemm_rowscale", code, a.data_ptr(), b.data_ptr(), scale.data_ptr(),
                  out_ptr, M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
                  stride_m, stride_n, stream)
    else:
        _hip.call("tk_gemm_swiglu", code, a.data_ptr(), b.data_ptr(), b2.data_ptr(), out_ptr,
                  M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1), b2.stride(0),
                  b2.stride(1), stride_m, stride_n, stream)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("entry", ["tk_gemm", "tk_gemm_rowscale", "tk_gemm_swiglu"])
@pytest.mark.parametrize(("pad", "col_stride", "offset"), LAYOUTS)
def test_strided_output_is_bitwise_the_contiguous_result(entry, dtype, pad, col_stride,
                                                         offset) -> None:
    a, b, b2, scale = _operands(dtype, seed=len(entry) + pad + 7 * col_stride + offset)
    ref = torch.empty(M, N, device="cuda", dtype=dtype)
    _call(entry, dtype, a, b, b2, scale, ref.data_ptr(), N, 1)

    row_stride = N * col_stride + pad
    size = offset + (M - 1) * row_stride + (N - 1) * col_stride + 1 + 64
    sentinel = torch.full((size,), -12345, device="cuda", dtype=_INT[dtype])
    storage = sentinel.clone().view(dtype)
    out = torch.as_strided(storage, (M, N), (row_stride, col_stride), offset)
    _call(entry, dtype, a, b, b2, scale, out.data_ptr(), row_stride, col_stride)
    torch.cuda.synchronize()

    assert bits_equal(out, ref)
    written = torch.zeros(size, dtype=torch.bool, device="cuda")
    torch.as_strided(written, (M, N), (row_stride, col_stride), offset).fill_(True)
    untouched = storage.view(_INT[dtype])[~written]
    assert torch.equal(untouched, sentinel[~written])
