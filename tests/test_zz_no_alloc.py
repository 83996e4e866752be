"""tk_rmsnorm_bwd_noalloc: the norm backward with its partial rows in library-owned memory.

The entry point runs the same stage-1 and stage-2 kernels as tk_rmsnorm_bwd_stage1 +
tk_rmsnorm_bwd_stage2 with the same group count, so dx and dw must be bitwise those of the
two-call path. Two calls in a row (the second smaller) check that the shared array's leftover
contents from the first call do not leak into the second; a problem beyond the array's size is
rejected before any launch.
"""

from __future__ import annotations

import pytest
import torch

from _helpers import bits_equal
from tklab import _hip
from tklab.kernels._norm_common import EPS
from tklab.kernels.residual_rms_norm import _launch_forward as _residual_forward
from tklab.kernels.rms_norm import (
    _launch_backward_stage1,
    _launch_backward_stage2,
    _make_backward_buffers,
)

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _problem(rows, cols, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(rows, cols, device="cuda", dtype=dtype, generator=g)
    r = torch.randn(rows, cols, device="cuda", dtype=dtype, generator=g)
    w = (1 + 0.02 * torch.randn(cols, device="cuda", generator=g)).to(dtype)
    dy = torch.randn(rows, cols, device="cuda", dtype=dtype, generator=g)
    dsum = torch.randn(rows, cols, device="cuda", dtype=dtype, generator=g)
    s = torch.empty_like(x)
    y = torch.empty_like(x)
    rstd = torch.empty(rows, device="cuda", dtype=torch.float32)
    _residual_forward(x, r, w, s, y, rstd, eps=EPS, store_residual=True, store_stats=True)
    return s, w, rstd, dy, dsum


def _noalloc(s, w, rstd, dy, incoming, group_size, out=None):
    dx, dw = out if out is not None else (torch.empty_like(s), torch.empty_like(w))
    _hip.call(
        "tk_rmsnorm_bwd_noalloc",
        _hip.dtype_code(s.dtype),
        dx.data_ptr(),
        dw.data_ptr(),
        dy.data_ptr(),
        _hip.ptr(incoming),
        s.data_ptr(),
        w.data_ptr(),
        rstd.data_ptr(),
        s.shape[0],
        s.shape[1],
        s.stride(0),
        dy.stride(0),
        0 if incoming is None else incoming.stride(0),
        dx.stride(0),
        group_size,
        _hip.stream_of(s),
    )
    return dx, dw


def _two_call(s, w, rstd, dy, incoming, group_size):
    buffers = _make_backward_buffers(s, w, group_size=group_size)
    _launch_backward_stage1(dy, s, w, rstd, buffers, incoming_dx=incoming)
    _launch_backward_stage2(buffers, s.shape[1])
    return buffers.dx, buffers.dw


CASES = [
    # (rows, cols, dtype, group_size, incoming): the first fills the array exactly
    # (512 x 8192 floats), each next one is smaller.
    (16384, 8192, torch.bfloat16, 512, True),
    (4099, 4096, torch.bfloat16, 512, False),
    (300, 1000, torch.float32, 512, True),
    (7, 16, torch.float16, 512, False),
]


def test_matches_the_two_call_backward_on_consecutive_calls() -> None:
    for i, (rows, cols, dtype, groups, with_incoming) in enumerate(CASES):
        print(f"noalloc case {i}: rows={rows} cols={cols} {dtype} groups={groups}", flush=True)
        s, w, rstd, dy, dsum = _problem(rows, cols, dtype, seed=100 + i)
        incoming = dsum if with_incoming else None
        got_dx, got_dw = _noalloc(s, w, rstd, dy, incoming, groups)
        torch.cuda.synchronize()
        want_dx, want_dw = _two_call(s, w, rstd, dy, incoming, groups)
        torch.cuda.synchronize()
        assert bits_equal(got_dx, want_dx), f"dx differs in case {i}"
        assert bits_equal(got_dw, want_dw), f"dw differs in case {i}"


def test_repeated_call_is_bitwise_stable_after_a_larger_one() -> None:
    big = _problem(2048, 4096, torch.bfloat16, seed=7)[:4]
    small = _problem(33, 4096, torch.bfloat16, seed=8)[:4]
    first = _noalloc(*small, None, 512)
    _noalloc(*big, None, 512)
    second = _noalloc(*small, None, 512)
    torch.cuda.synchronize()
    assert bits_equal(first[0], second[0])
    assert bits_equal(first[1], second[1])


def test_rejects_problems_beyond_the_scratch_array() -> None:
    s, w, rstd, dy, _ = _problem(1024, 16384, torch.bfloat16, seed=9)
    with pytest.raises(_hip.HipLibraryError, match="scratch"):
        _noalloc(s, w, rstd, dy, None, 512)
    # 256 groups x 16384 columns fill the array exactly and are accepted.
    got = _noalloc(s, w, rstd, dy, None, 256)
    want = _two_call(s, w, rstd, dy, None, 256)
    torch.cuda.synchronize()
    assert bits_equal(got[0], want[0])
    assert bits_equal(got[1], want[1])
    assert 256 * 16384 * 4 == SCRATCH_BYTES


def test_graph_capture_replays_match_the_two_call_backward() -> None:
    """The use the entry point exists for: one call captured in a HIP graph (after a warm-up
    call that sets up the device array), replayed with new inputs copied into the captured
    tensors, eager work and a synchronization between replays; every replay's dx and dw are
    bitwise those of the two-call path on the same inputs."""
    rows, cols, groups = 1000, 4096, 256
    s, w, rstd, dy, dsum = _problem(rows, cols, torch.bfloat16, seed=20)
    out = (torch.empty_like(s), torch.empty_like(w))
    _noalloc(s, w, rstd, dy, dsum, groups, out)  # warm-up: device array set up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _noalloc(s, w, rstd, dy, dsum, groups, out)
    torch.cuda.synchronize()
    for replay in range(3):
        print(f"noalloc graph replay {replay}", flush=True)
        fresh = _problem(rows, cols, torch.bfloat16, seed=21 + replay)
        for captured, new in zip((s, w, rstd, dy, dsum), fresh):
            captured.copy_(new)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_dx, want_dw = _two_call(s, w, rstd, dy, dsum, groups)
        torch.cuda.synchronize()
        assert bits_equal(out[0], want_dx), f"dx differs on replay {replay}"
        assert bits_equal(out[1], want_dw), f"dw differs on replay {replay}"
