"""Calibration kernels behind bench.py's measured roofs (no reference counterpart)."""

from __future__ import annotations

import pytest
import torch

from tklab import _hip

pytestmark = pytest.mark.gpu


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("nbytes", [16, 48, 4096 * 16 + 16, (1 << 24) + 4096 * 16 * 3 + 32])
def test_roof_copy_is_an_exact_copy(nbytes: int) -> None:
    g = torch.Generator(device="cuda").manual_seed(nbytes % 1000)
    src = torch.randint(-(2**31), 2**31 - 1, (nbytes // 4 + 4,), device="cuda",
                        dtype=torch.int32, generator=g)
    dst = torch.full_like(src, -1)
    _hip.call("tk_roof_copy", src.data_ptr(), dst.data_ptr(), nbytes, _stream())
    torch.cuda.synchronize()
    n = nbytes // 4
    assert torch.equal(dst[:n], src[:n])
    assert bool((dst[n:] == -1).all())


@pytest.mark.parametrize("code", [1, 2])
def test_roof_mfma_is_finite_and_deterministic(code: int) -> None:
    out = torch.empty(1024, device="cuda")
    _hip.call("tk_roof_mfma", code, out.data_ptr(), 1024, 64, _stream())
    first = out.clone()
    _hip.call("tk_roof_mfma", code, out.data_ptr(), 1024, 64, _stream())
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    assert bool((out != 0).any())
    assert torch.equal(out, first)


def test_roof_arguments_are_checked() -> None:
    out = torch.empty(8, device="cuda")
    with pytest.raises(_hip.HipLibraryError, match="multiple of 16"):
        _hip.call("tk_roof_copy", out.data_ptr(), out.data_ptr(), 20, _stream())
    with pytest.raises(_hip.HipLibraryError, match="multiple of 4"):
        _hip.call("tk_roof_mfma", 1, out.data_ptr(), 6, 8, _stream())
    with pytest.raises(_hip.HipLibraryError, match="multiple of 8"):
        _hip.call("tk_roof_mfma", 1, out.data_ptr(), 8, 12, _stream())
    with pytest.raises(_hip.HipLibraryError, match="dtype"):
        _hip.call("tk_roof_mfma", 0, out.data_ptr(), 8, 8, _stream())
