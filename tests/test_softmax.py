"""GPU parity of tk_softmax_fwd against the CPU oracle and torch.softmax."""

from __future__ import annotations

import pytest
import torch

from _helpers import dev, host, name
from oracle import oracle
from tklab.harness.tolerances import assert_close, assert_relative_frobenius
from tklab.kernels.fused_softmax import _launch, softmax

pytestmark = pytest.mark.gpu


def _check(x: torch.Tensor) -> None:
    y = softmax(x)
    expected = dev(oracle.softmax(host(x), name(x.dtype)), y)
    # Tolerances of the dtype table (float32: rtol 1e-4, atol 1e-5).
    assert_close(y, expected)
    assert_close(y, torch.softmax(x.float(), dim=-1))


def test_config_shape_float32_4096x4096() -> None:
    torch.manual_seed(0)
    x = torch.randn(4096, 4096, device="cuda")
    y = softmax(x)
    expected = dev(oracle.softmax(host(x), "float32"), y)
    assert_close(y, expected)
    assert_relative_frobenius(y, expected, max_relative_error=1e-5)
    rows = y.double().sum(dim=1)
    torch.testing.assert_close(rows, torch.ones_like(rows), rtol=0, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [1, 3, 64, 128, 1000, 1024, 4096, 4097, 8192, 16384, 65536])
def test_widths_and_dtypes(dtype: torch.dtype, cols: int) -> None:
    torch.manual_seed(cols)
    _check(torch.randn(37, cols, device="cuda", dtype=dtype))


@pytest.mark.parametrize(("rows", "cols", "dtype"), [(4097, 1000, torch.float32), (4099, 4096, torch.bfloat16), (5000, 64, torch.float16)])
def test_two_rows_per_wave_with_an_odd_row_count(rows, cols, dtype) -> None:
    """From 4096 rows on, single-wave rows go two to a wave; an odd count leaves the last
    wave one row, which it loads twice and stores once."""
    torch.manual_seed(rows)
    x = torch.randn(rows, cols, device="cuda", dtype=dtype)
    out_storage = torch.full((rows + 1, cols), 7.0, device="cuda", dtype=dtype)
    _launch((x,), out_storage[:rows])
    assert torch.all(out_storage[rows] == 7.0)
    expected = dev(oracle.softmax(host(x), name(dtype)), x)
    assert_close(out_storage[:rows], expected)


def test_row_strided_adversarial_view() -> None:
    torch.manual_seed(0)
    x = torch.randn(64, 1000, device="cuda")[::2]
    _check(x)


def test_misaligned_base_uses_the_scalar_path() -> None:
    torch.manual_seed(1)
    storage = torch.randn(33 * 512 + 1, device="cuda")
    x = storage[1:].view(33, 512)
    _check(x)


def test_launch_writes_into_a_strided_output() -> None:
    torch.manual_seed(2)
    x = torch.randn(16, 256, device="cuda")
    out_storage = torch.full((16, 512), 7.0, device="cuda")
    out = out_storage[:, :256]
    _launch((x,), out)
    assert_close(out, torch.softmax(x, dim=-1))
    assert torch.all(out_storage[:, 256:] == 7.0)


def test_constant_rows_are_uniform_and_large_values_stay_finite() -> None:
    x = torch.full((4, 1000), 3.0, device="cuda")
    x[1] = 1e30
    x[2, :500] = -1e30
    y = softmax(x)
    assert torch.isfinite(y).all()
    torch.testing.assert_close(y[0], torch.full_like(y[0], 1e-3), rtol=1e-6, atol=0)
    torch.testing.assert_close(y[2, 500:], torch.full_like(y[2, 500:], 2e-3), rtol=1e-6, atol=0)
    assert torch.all(y[2, :500] == 0)


# ---------------------------------------------------------------- online softmax


def _check_online(x: torch.Tensor) -> None:
    from tklab.kernels.fused_softmax import online_softmax

    y = online_softmax(x)
    expected = dev(oracle.softmax(host(x), name(x.dtype)), y)
    assert_close(y, expected)
    assert_close(y, torch.softmax(x.float(), dim=-1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("cols", [1, 1000, 16384, 16385, 65536, 65537, 200003])
def test_online_widths_and_dtypes(dtype: torch.dtype, cols: int) -> None:
    """Chunk edges (16384, 16385), the single-pass limit and past it, ragged tails."""
    torch.manual_seed(cols + 7)
    _check_online(torch.randn(5, cols, device="cuda", dtype=dtype))


def test_online_matches_single_pass_where_both_apply() -> None:
    from tklab.kernels.fused_softmax import online_softmax

    torch.manual_seed(8)
    x = torch.randn(64, 4096, device="cuda")
    y1 = softmax(x)
    y2 = online_softmax(x)
    # One chunk per row: the same maximum, a sum over the same values.
    torch.testing.assert_close(y2, y1, rtol=1e-6, atol=1e-9)


def test_online_wide_row_sums_to_one_and_is_deterministic() -> None:
    from tklab.kernels.fused_softmax import online_softmax

    torch.manual_seed(9)
    x = torch.randn(3, 1 << 21, device="cuda") * 4
    x[1, 123456] = 80.0  # one dominant entry, far from the chunk holding the others
    y = online_softmax(x)
    rows = y.double().sum(dim=1)
    torch.testing.assert_close(rows, torch.ones_like(rows), rtol=0, atol=1e-4)
    assert_close(y, torch.softmax(x, dim=-1))
    assert torch.equal(online_softmax(x), y)


def test_online_single_read_chunk_limit_and_many_rows() -> None:
    """Exactly 64 chunks per row (the widest single-read row), one column more (the two-launch
    path), and 256 rows of 7 chunks (1792 workgroups, many rows in flight at once)."""
    torch.manual_seed(11)
    _check_online(torch.randn(2, 1 << 20, device="cuda"))
    _check_online(torch.randn(2, (1 << 20) + 1, device="cuda", dtype=torch.bfloat16))
    _check_online(torch.randn(256, 100000, device="cuda"))


@pytest.mark.parametrize(("rows", "cols", "dtype"), [
    (5, 200003, torch.float32), (3, 1 << 20, torch.bfloat16), (7, 70001, torch.float16),
])
def test_online_single_read_fallback_gives_the_same_bits(rows, cols, dtype, monkeypatch) -> None:
    """With its bounded wait set to zero polls every workgroup computes its row's partials from
    x itself; the result must be bitwise that of the exchange through the workspace."""
    from tklab.kernels.fused_softmax import online_softmax

    torch.manual_seed(rows + cols)
    x = torch.randn(rows, cols, device="cuda", dtype=dtype) * 3
    exchanged = online_softmax(x)
    monkeypatch.setenv("TKLAB_ONLINE_SOFTMAX_POLLS", "0")
    recomputed = online_softmax(x)
    torch.cuda.synchronize()
    assert torch.equal(recomputed, exchanged)
    assert_close(exchanged, torch.softmax(x.float(), dim=-1).to(dtype))


def test_online_single_read_replays_in_a_graph() -> None:
    """The single-read call (workspace clear + kernel, no memset) captured once and replayed on
    new inputs, with eager calls and synchronizations between replays: every replay matches
    the eager call bitwise."""
    from tklab.kernels.fused_softmax import _launch_online

    x = torch.randn(8, 300000, device="cuda")
    y = torch.empty_like(x)
    _launch_online((x,), y)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _launch_online((x,), y)
    for seed in range(3):
        gen = torch.Generator(device="cuda").manual_seed(40 + seed)
        x.copy_(torch.randn(x.shape, device="cuda", generator=gen) * (seed + 1))
        graph.replay()
        torch.cuda.synchronize()
        eager = torch.empty_like(x)
        _launch_online((x,), eager)
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        assert_close(y, torch.softmax(x, dim=-1))


def test_online_strided_misaligned_and_masked_rows() -> None:
    from tklab.kernels.fused_softmax import _launch_online

    torch.manual_seed(10)
    x = torch.randn(6, 2 * 70001, device="cuda")[:, 1:70002]  # misaligned, scalar path
    _check_online(x)
    x = torch.randn(4, 40000, device="cuda")
    x[0, :20000] = -torch.inf  # whole chunks of -inf contribute nothing
    x[2] = -1e30
    out_storage = torch.full((4, 50000), 7.0, device="cuda")
    out = out_storage[:, :40000]
    _launch_online((x,), out)
    assert_close(out, torch.softmax(x, dim=-1))
    assert torch.all(out[0, :20000] == 0)
    assert torch.all(out_storage[:, 40000:] == 7.0)
