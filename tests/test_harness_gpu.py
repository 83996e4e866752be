"""GPU runs of the benchmark harness: the registry runner on a reduced spec, and a
short peak calibration that round-trips through the cache validation."""

from __future__ import annotations

import dataclasses
from pathlib import Path

import pytest
import torch

from tklab.harness import roofline
from tklab.harness.bench import bench_spec
from tklab.harness.jsonio import read_json_object
from tklab.harness.timing import time_ms
from tklab.kernels.fused_softmax import SOFTMAX
from tklab.kernels.matmul import MATMUL_FP32ACC

pytestmark = pytest.mark.gpu


def test_timer_quantiles_are_ordered_and_track_the_work() -> None:
    x = torch.randn(1 << 24, device="cuda")
    small = time_ms(lambda: x[: 1 << 20].mul_(1.0), warmup_ms=5, repetition_ms=20)
    lo, mid, hi = time_ms(lambda: x.mul_(1.0), warmup_ms=5, repetition_ms=20,
                          quantiles=[0.2, 0.5, 0.8])
    assert 0 < lo <= mid <= hi
    assert mid > small


def test_bench_spec_rows_carry_the_roofline_metrics() -> None:
    softmax = dataclasses.replace(SOFTMAX, sizes=(1024,), dtypes=(torch.float32,))
    rows = bench_spec(softmax, peak_bw_gbps=5880.0, cublas_tflops=None, theoretical_tflops=None,
                      warmup_ms=5, repetition_ms=20)
    assert len(rows) == 1
    row = rows[0]
    assert row["kernel"] == "fused_softmax" and row["size"] == 1024 and row["dtype"] == "float32"
    assert 0 < row["ms_lo"] <= row["ms"] <= row["ms_hi"]
    assert row["gbps"] > 0 and row["pct_peak"] == pytest.approx(100 * row["gbps"] / 5880.0)
    assert row["naive_ms"] > 0 and isinstance(row["reference_baseline"], str)
    gemm = dataclasses.replace(MATMUL_FP32ACC, sizes=(1024,), dtypes=(torch.float16,))
    row = bench_spec(gemm, peak_bw_gbps=None, cublas_tflops=1300.0, theoretical_tflops=2516.6,
                     warmup_ms=5, repetition_ms=20)[0]
    assert row["tflops"] > 0 and row["reference_tflops"] > 0
    assert row["pct_theoretical"] == pytest.approx(100 * row["tflops"] / 2516.6)


def test_short_calibration_round_trips_through_the_cache(tmp_path: Path, monkeypatch) -> None:
    arch = torch.cuda.get_device_properties(0).gcnArchName
    if "gfx950" not in arch:
        pytest.skip(f"no audited profile for {arch!r}")
    peaks = roofline.measure_peaks(0, bw_element_counts=(1 << 24,), tflops_sizes=(2048,),
                                   warmup_ms=5, repetition_ms=20)
    assert peaks["peak_bw_gbps"] > 1000
    assert peaks["cublas_tflops_fp16_fp32acc"] > 100
    clock = peaks["theoretical_ceiling_sm_clock_mhz"]
    assert 500 <= clock <= 3000
    assert peaks["theoretical_tflops_fp16_fp32acc_at_measured_clock"] == pytest.approx(
        roofline.theoretical_tflops_fp16_fp32acc(clock)
    )
    path = tmp_path / "peaks.json"
    monkeypatch.setattr(roofline, "measure_peaks", lambda device=0: peaks)
    first = roofline.load_or_measure_peaks(path)
    assert read_json_object(path)["peak_bw_gbps"] == first["peak_bw_gbps"]
    # A second load reuses the cache only after its provenance validates.
    monkeypatch.setattr(roofline, "measure_peaks", lambda device=0: pytest.fail("re-measured"))
    assert roofline.load_or_measure_peaks(path)["tflops_samples"] == peaks["tflops_samples"]
