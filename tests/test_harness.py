"""CPU tests of the benchmark harness: JSON persistence, roofline formulas and
profiles, cached-peaks validation, and benchmark-row metric semantics (the
behaviour the reference pins in tests/test_jsonio.py, test_roofline.py and
test_bench.py)."""

from __future__ import annotations

import copy
from pathlib import Path

import pytest
import torch

import tklab.kernels  # noqa: F401  (registers every spec)
from tklab.harness.bench import (
    BenchRow,
    _add_performance_metrics,
    _compose_row,
    _Timings,
    _validate_benchmark_request,
)
from tklab.harness.jsonio import JsonObject, read_json_object, write_json_atomic
from tklab.harness.roofline import (
    MI355X_PROFILE,
    PEAKS_SCHEMA_VERSION,
    RTX4060_PROFILE,
    TflopsSample,
    _maximum_observed_sm_clock_mhz,
    _profile_for,
    _validate_stored_peaks,
    theoretical_tflops_fp16_fp16acc,
    theoretical_tflops_fp16_fp32acc,
)
from tklab.harness.timing import time_ms
from tklab.kernels.fused_softmax import SOFTMAX
from tklab.kernels.matmul import MATMUL_FP32ACC
from tklab.registry import REGISTRY

# ---------------------------------------------------------------- jsonio


def test_json_round_trip_and_no_leftover_temporaries(tmp_path: Path) -> None:
    path = tmp_path / "sub" / "result.json"
    payload: JsonObject = {"schema_version": 1, "rows": [{"size": 128, "gbps": 42.0}]}
    write_json_atomic(path, payload)
    write_json_atomic(path, payload)  # replacing an existing file
    assert read_json_object(path) == payload
    assert [p.name for p in path.parent.iterdir()] == ["result.json"]


def test_read_json_object_rejects_top_level_array(tmp_path: Path) -> None:
    path = tmp_path / "array.json"
    path.write_text("[]", encoding="utf-8")
    with pytest.raises(ValueError, match="top-level"):
        read_json_object(path)


def test_read_json_object_rejects_invalid_json(tmp_path: Path) -> None:
    path = tmp_path / "bad.json"
    path.write_text("{", encoding="utf-8")
    with pytest.raises(ValueError, match="invalid JSON"):
        read_json_object(path)


# ---------------------------------------------------------------- roofline


def test_mi355x_rated_ceiling_is_the_published_dense_fp16_peak() -> None:
    """256 CU x 4 matrix SIMDs x 1024 FLOP/clk x 2400 MHz: AMD's 2.5 PFLOP/s (2516.6)."""
    assert theoretical_tflops_fp16_fp32acc(MI355X_PROFILE.rated_boost_mhz) == pytest.approx(
        2516.5824
    )
    assert _profile_for("AMD Instinct MI355X") is MI355X_PROFILE
    assert _profile_for("AMD Radeon Graphics", "gfx950:sramecc+:xnack-") is MI355X_PROFILE


def test_rtx4060_rated_ceiling_matches_the_reference() -> None:
    """The reference's audited 30.22848 TFLOP/s at 2460 MHz."""
    assert theoretical_tflops_fp16_fp32acc(
        RTX4060_PROFILE.rated_boost_mhz, profile=RTX4060_PROFILE
    ) == pytest.approx(30.22848)


def test_fp16_accumulate_ceiling_per_architecture() -> None:
    """CDNA4 MFMA accumulates in float32 only; Ada doubles FP16-accumulate throughput."""
    clock = 2100
    assert theoretical_tflops_fp16_fp16acc(clock) == pytest.approx(
        theoretical_tflops_fp16_fp32acc(clock)
    )
    assert theoretical_tflops_fp16_fp16acc(clock, profile=RTX4060_PROFILE) == pytest.approx(
        2 * theoretical_tflops_fp16_fp32acc(clock, profile=RTX4060_PROFILE)
    )


def test_unknown_gpu_has_no_profile() -> None:
    with pytest.raises(ValueError, match="no theoretical compute profile"):
        _profile_for("Some Other GPU")


def _clock_sample(clock_mhz: int) -> TflopsSample:
    return {"n": 1024, "ms": 1.0, "tflops": 1.0, "sm_clock_mhz": clock_mhz,
            "sm_clock_min_mhz": clock_mhz, "sm_clock_max_mhz": clock_mhz,
            "sm_clock_samples_mhz": [clock_mhz]}


def test_theoretical_ceiling_uses_the_maximum_clock_across_sweeps() -> None:
    assert _maximum_observed_sm_clock_mhz([_clock_sample(2105)], [_clock_sample(2400)]) == 2400
    with pytest.raises(ValueError, match="at least one"):
        _maximum_observed_sm_clock_mhz([], [])


def _cached_peaks() -> JsonObject:
    return {
        "schema_version": PEAKS_SCHEMA_VERSION,
        "gpu_name": "AMD Instinct MI355X",
        "compute_capability": "9.5",
        "torch_version": "2.10.0+rocm7.0",
        "triton_version": "tklab_hip abi 1",
        "calibration_started_at_utc": "2026-12-01T12:00:00+00:00",
        "calibration_preflight_gpu_utilization_pct": [0, 0, 1, 0, 0],
        "calibration_preflight_gpu_utilization_limit_pct": 10,
        "peak_bw_gbps": 5880.0,
        "cublas_tflops_fp16_fp32acc": 1330.0,
        "theoretical_tflops_fp16_fp32acc_at_measured_clock": 2516.6,
        "theoretical_tflops_fp16_fp16acc_at_measured_clock": 2516.6,
        "theoretical_ceiling_sm_clock_mhz": 2400,
        "theoretical_provenance": {
            "model": "AMD Instinct MI355X",
            "rated_boost_clock_mhz": 2400,
            "streaming_multiprocessors": 256,
            "tensor_cores_per_sm": 4,
            "fp16_fp32acc_flops_per_clock_per_tensor_core": 1024,
            "fp16_fp32acc_rated_tflops": 2516.5824,
            "fp16_fp16acc_rated_tflops": 2516.5824,
            "ceiling_clock_policy": "maximum observed clock",
            "product_spec_url": "https://example.com/product",
            "architecture_whitepaper_url": "https://example.com/architecture",
        },
    }


_ENV = {
    "expected_gpu_name": "AMD Instinct MI355X",
    "expected_compute_capability": "9.5",
    "expected_torch_version": "2.10.0+rocm7.0",
    "expected_triton_version": "tklab_hip abi 1",
}


def test_cached_peaks_accept_matching_environment() -> None:
    _validate_stored_peaks(_cached_peaks(), path=Path("peaks.json"), **_ENV)


def test_cached_peaks_reject_stale_software_stack() -> None:
    env = dict(_ENV, expected_torch_version="2.11.0+rocm7.1")
    with pytest.raises(ValueError, match=r"active environment.*torch_version"):
        _validate_stored_peaks(_cached_peaks(), path=Path("peaks.json"), **env)
    env = dict(_ENV, expected_triton_version="tklab_hip abi 2")
    with pytest.raises(ValueError, match=r"active environment.*triton_version"):
        _validate_stored_peaks(_cached_peaks(), path=Path("peaks.json"), **env)


@pytest.mark.parametrize(
    "field,value,message",
    [
        ("peak_bw_gbps", 0.0, "invalid positive numeric fields"),
        ("cublas_tflops_fp16_fp32acc", float("nan"), "invalid positive numeric fields"),
        ("theoretical_ceiling_sm_clock_mhz", True, "invalid positive numeric fields"),
        ("schema_version", PEAKS_SCHEMA_VERSION - 1, "incompatible peaks schema"),
        ("calibration_preflight_gpu_utilization_pct", [0, 55], "utilization limit"),
        ("calibration_preflight_gpu_utilization_pct", [], "utilization samples"),
        ("calibration_preflight_gpu_utilization_limit_pct", 101, "utilization limit"),
        ("theoretical_provenance", [], "must be an object"),
    ],
)
def test_cached_peaks_reject_corrupt_payloads(field: str, value: object, message: str) -> None:
    payload = _cached_peaks()
    payload[field] = value
    with pytest.raises(ValueError, match=message):
        _validate_stored_peaks(payload, path=Path("peaks.json"), **_ENV)


def test_cached_peaks_reject_missing_fields() -> None:
    payload = _cached_peaks()
    del payload["peak_bw_gbps"]
    with pytest.raises(ValueError, match="missing required fields: peak_bw_gbps"):
        _validate_stored_peaks(payload, path=Path("peaks.json"), **_ENV)
    payload = _cached_peaks()
    provenance = copy.deepcopy(payload["theoretical_provenance"])
    del provenance["tensor_cores_per_sm"]
    payload["theoretical_provenance"] = provenance
    with pytest.raises(ValueError, match="provenance is missing fields: tensor_cores_per_sm"):
        _validate_stored_peaks(payload, path=Path("peaks.json"), **_ENV)


# ---------------------------------------------------------------- bench metrics


def _row(kernel: str, ms: float, torch_ms: float) -> BenchRow:
    return {"kernel": kernel, "dtype": "float16", "size": 512, "ms": ms, "ms_lo": ms,
            "ms_hi": ms, "torch_ms": torch_ms, "speedup": torch_ms / ms}


def test_compute_metrics_separate_same_size_blas_from_peak() -> None:
    row = _row("matmul_fp32acc", 0.04, 0.02)
    _add_performance_metrics(row, spec=MATMUL_FP32ACC, size=512, dtype=torch.float16,
                             milliseconds=0.04, peak_bw_gbps=None, cublas_tflops=32.0,
                             theoretical_tflops=64.0)
    flops = 2 * 512**3
    assert row["tflops"] == pytest.approx(flops / 0.04e-3 / 1e12)
    assert row["reference_tflops"] == pytest.approx(2 * row["tflops"])
    assert row["pct_theoretical"] == pytest.approx(100 * row["tflops"] / 64.0)
    assert row["pct_cublas_same_size"] == pytest.approx(50.0)
    assert row["pct_cublas_peak"] == pytest.approx(100.0 * row["tflops"] / 32.0)
    assert "gbps" not in row


def test_compute_metrics_without_a_blas_roof() -> None:
    row = _row("matmul_fp32acc", 0.04, 0.02)
    _add_performance_metrics(row, spec=MATMUL_FP32ACC, size=512, dtype=torch.float16,
                             milliseconds=0.04, peak_bw_gbps=None, cublas_tflops=None,
                             theoretical_tflops=64.0)
    assert "pct_cublas_peak" not in row and "pct_cublas_same_size" not in row


def test_memory_metrics_price_the_cost_model_against_the_bandwidth_roof() -> None:
    row = _row("softmax", 0.05, 0.1)
    _add_performance_metrics(row, spec=SOFTMAX, size=4096, dtype=torch.float32,
                             milliseconds=0.05, peak_bw_gbps=5000.0, cublas_tflops=None,
                             theoretical_tflops=None)
    assert SOFTMAX.bytes_moved is not None
    gbps = SOFTMAX.bytes_moved(4096, torch.float32) / 0.05e-3 / 1e9
    assert row["gbps"] == pytest.approx(gbps)
    assert row["pct_peak"] == pytest.approx(100 * gbps / 5000.0)


def test_missing_roofs_are_errors() -> None:
    with pytest.raises(ValueError, match="bandwidth peak"):
        _add_performance_metrics(_row("softmax", 1, 1), spec=SOFTMAX, size=4096,
                                 dtype=torch.float32, milliseconds=1.0, peak_bw_gbps=None,
                                 cublas_tflops=None, theoretical_tflops=None)
    with pytest.raises(ValueError, match="theoretical peak"):
        _add_performance_metrics(_row("matmul_fp32acc", 1, 1), spec=MATMUL_FP32ACC, size=512,
                                 dtype=torch.float16, milliseconds=1.0, peak_bw_gbps=None,
                                 cublas_tflops=32.0, theoretical_tflops=None)


@pytest.mark.parametrize("name", sorted(REGISTRY))
def test_rows_keep_their_identity_under_every_specs_metadata(name: str) -> None:
    """bench_spec lays each spec's benchmark metadata under the row's identity fields, so
    a metadata key such as the HIP kernel's name never renames the row (the reference's
    plots group rows by row["kernel"])."""
    spec = REGISTRY[name]
    dtype, size = spec.dtypes[0], spec.sizes[0]
    timings = _Timings(ms=0.5, ms_lo=0.4, ms_hi=0.6, torch_ms=1.0, naive_ms=2.0)
    row = _compose_row(spec, size=size, dtype=dtype, timings=timings, peak_bw_gbps=5000.0,
                       cublas_tflops=1000.0, theoretical_tflops=2500.0)
    assert row["kernel"] == spec.name
    assert (row["dtype"], row["size"]) == (str(dtype).removeprefix("torch."), size)
    assert (row["ms"], row["ms_lo"], row["ms_hi"], row["torch_ms"]) == (0.5, 0.4, 0.6, 1.0)
    assert row["speedup"] == pytest.approx(2.0) and row["speedup_vs_naive"] == pytest.approx(4.0)
    if spec.benchmark_metadata is not None:
        for key, value in spec.benchmark_metadata(size, dtype).items():
            if key not in ("kernel", "dtype", "size"):
                assert row[key] == value
    assert ("gbps" in row) == (spec.bound == "memory")
    assert ("tflops" in row) == (spec.bound == "compute")


def test_benchmark_request_validation_runs_before_any_gpu_work() -> None:
    with pytest.raises(ValueError, match="device index must be non-negative"):
        _validate_benchmark_request(device=-1, warmup_ms=25, repetition_ms=100)
    with pytest.raises(ValueError, match="warmup_ms must be positive.*repetition_ms"):
        _validate_benchmark_request(device=0, warmup_ms=0, repetition_ms=-1)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="sees 0"):
            _validate_benchmark_request(device=0, warmup_ms=25, repetition_ms=100)


def test_timer_rejects_bad_parameters_before_touching_a_gpu() -> None:
    with pytest.raises(ValueError, match="positive"):
        time_ms(lambda: None, warmup_ms=0)
    with pytest.raises(ValueError, match=r"\[0, 1\]"):
        time_ms(lambda: None, quantiles=[0.5, 1.5])


def test_rocm_smi_clock_and_use_lines_parse(monkeypatch) -> None:
    """The sclk level field is a number or ``S``; both forms give the MHz value."""
    import subprocess
    from types import SimpleNamespace

    from tklab.harness import roofline

    outputs = {
        "--showclocks": "GPU[0]\t\t: mclk clock level: 0: (2000Mhz)\n"
                        "GPU[0]\t\t: sclk clock level: S: (2104Mhz)\n",
        "--showuse": "GPU[0]\t\t: GPU use (%): 7\n",
    }

    def fake_run(cmd, **kwargs):
        return SimpleNamespace(stdout=outputs[cmd[-1]])

    monkeypatch.setattr(subprocess, "run", fake_run)
    assert roofline._sm_clock_mhz(0) == 2104
    assert roofline.gpu_utilization_pct(0) == 7
    outputs["--showclocks"] = "GPU[0]\t\t: sclk clock level: 3: (1900Mhz)\n"
    assert roofline._sm_clock_mhz(0) == 1900
    outputs["--showuse"] = "no such line\n"
    with pytest.raises(RuntimeError, match="utilization"):
        roofline.gpu_utilization_pct(0)
