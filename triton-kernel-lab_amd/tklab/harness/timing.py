"""GPU timing for the registry benchmarks and the peak calibration.

The role ``triton.testing.do_bench`` plays in the reference
(``src/tklab/harness/bench.py:98-103``): launch a callable for about ``warmup_ms``,
then time about ``repetition_ms`` worth of single launches with HIP events on the
current stream. Before each timed launch a 256 MiB buffer is cleared (the size of
MI355X's last-level cache), so no launch reads what the previous one left cached.
"""

from __future__ import annotations

import statistics
from collections.abc import Callable, Sequence

import torch

_FLUSH_BYTES = 256 << 20
_flush_buffers: dict[torch.device, torch.Tensor] = {}


def _flush_buffer(device: torch.device) -> torch.Tensor:
    buf = _flush_buffers.get(device)
    if buf is None:
        buf = torch.empty(_FLUSH_BYTES // 4, dtype=torch.int32, device=device)
        _flush_buffers[device] = buf
    return buf


def _quantile(sorted_ms: Sequence[float], q: float) -> float:
    """Linear-interpolation quantile of an ascending sequence."""
    pos = q * (len(sorted_ms) - 1)
    lo = int(pos)
    hi = min(lo + 1, len(sorted_ms) - 1)
    return sorted_ms[lo] + (sorted_ms[hi] - sorted_ms[lo]) * (pos - lo)


def time_ms(
    fn: Callable[[], object],
    *,
    warmup_ms: float = 25,
    repetition_ms: float = 100,
    quantiles: Sequence[float] | None = None,
    device: torch.device | None = None,
) -> float | list[float]:
    """Median launch time of ``fn`` in ms, or the requested ``quantiles``.

    Raises:
        ValueError: If a duration is not positive or a quantile is outside [0, 1].
    """
    if warmup_ms <= 0 or repetition_ms <= 0:
        raise ValueError("warmup and repetition durations must be positive")
    if quantiles is not None and any(not 0.0 <= q <= 1.0 for q in quantiles):
        raise ValueError("quantiles must lie in [0, 1]")
    device = device or torch.device("cuda", torch.cuda.current_device())
    flush = _flush_buffer(device)
    stream = torch.cuda.current_stream(device)

    # Estimate one launch from five (events around the launch only, not the flush), then
    # size the warmup and the timed set.
    fn()
    torch.cuda.synchronize(device)
    probes = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(5)]
    for a, b in probes:
        flush.zero_()
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize(device)
    estimate = max(statistics.fmean(a.elapsed_time(b) for a, b in probes), 1e-3)
    for _ in range(max(1, int(warmup_ms / estimate))):
        fn()
    reps = max(1, int(repetition_ms / estimate))
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
    for a, b in events:
        flush.zero_()
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize(device)
    times = sorted(a.elapsed_time(b) for a, b in events)
    if quantiles is None:
        return float(statistics.median(times))
    return [float(_quantile(times, q)) for q in quantiles]
