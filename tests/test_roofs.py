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


@pytest.mark.parametrize("reads,writes", [(1, 0), (0, 1), (1, 1), (2, 1), (3, 1), (2, 2), (3, 2)])
@pytest.mark.parametrize("policy,tile,grid", [(0, 16, 0), (1, 8, 0), (0, 8, 3)])
@pytest.mark.parametrize("nbytes", [65536 * 16, 65536 * 3 + 4096 + 48])
def test_roof_stream_writes_the_xor_of_its_reads(reads: int, writes: int, policy: int, tile: int,
                                                 grid: int, nbytes: int) -> None:
    """Written chunk i is {i, 0, 0, 0} xor the chunks read at position i, for whole and
    partial tiles, one workgroup per tile or a 3-workgroup grid-stride walk; nothing past
    `bytes` of any destination array is written."""
    g = torch.Generator(device="cuda").manual_seed(reads * 10 + writes)
    chunks = nbytes // 16
    src = torch.randint(-(2**31), 2**31 - 1, (max(reads, 1) * chunks * 4,), device="cuda",
                        dtype=torch.int32, generator=g)
    dst = torch.full((max(writes, 1) * chunks * 4 + 64,), -1, device="cuda", dtype=torch.int32)
    _hip.call("tk_roof_stream", src.data_ptr(), dst.data_ptr(), nbytes, reads, writes, policy,
              tile, grid, _stream())
    torch.cuda.synchronize()
    want = torch.zeros(chunks, 4, device="cuda", dtype=torch.int32)
    want[:, 0] = torch.arange(chunks, device="cuda", dtype=torch.int32)
    for r in range(reads):
        want ^= src[r * chunks * 4:(r + 1) * chunks * 4].view(chunks, 4)
    for w in range(writes):
        assert torch.equal(dst[w * chunks * 4:(w + 1) * chunks * 4].view(chunks, 4), want)
    if writes == 0:
        assert bool((dst == -1).all())  # the sink store never fires on this data
    else:
        assert bool((dst[writes * chunks * 4:] == -1).all())


def test_roof_stream_arguments_are_checked() -> None:
    out = torch.empty(1 << 16, device="cuda")
    with pytest.raises(_hip.HipLibraryError, match="store_policy"):
        _hip.call("tk_roof_stream", out.data_ptr(), out.data_ptr(), 4096, 1, 1, 2, 16, 0, _stream())
    with pytest.raises(_hip.HipLibraryError, match="tile_kib"):
        _hip.call("tk_roof_stream", out.data_ptr(), out.data_ptr(), 4096, 1, 1, 0, 32, 0, _stream())
    with pytest.raises(_hip.HipLibraryError, match="max_workgroups"):
        _hip.call("tk_roof_stream", out.data_ptr(), out.data_ptr(), 4096, 1, 1, 0, 16, -1, _stream())
    with pytest.raises(_hip.HipLibraryError, match="unsupported mix"):
        _hip.call("tk_roof_stream", out.data_ptr(), out.data_ptr(), 4096, 1, 2, 0, 16, 0, _stream())
    with pytest.raises(_hip.HipLibraryError, match="read-only run"):
        _hip.call("tk_roof_stream", out.data_ptr(), out.data_ptr(), 16, 1, 0, 0, 16, 0, _stream())
