"""Roofline calibration: measured bandwidth and BLAS peaks, theoretical ceilings.

Contract of ``src/tklab/harness/roofline.py`` on MI355X:

- ``GpuTheoreticalProfile`` holds the audited hardware facts behind a clock-scaled
  dense FP16 ceiling. The reference's field names are kept with their CDNA meaning:
  ``streaming_multiprocessors`` = compute units, ``tensor_cores_per_sm`` = matrix-core
  SIMDs per CU, ``fp16_fp32acc_flops_per_clock_per_tensor_core`` = dense FP16 MFMA
  FLOP per clock per SIMD. ``MI355X_PROFILE`` is the default: 256 CU x 4 x 1024 x
  2400 MHz = 2516.58 TFLOP/s. CDNA4 MFMA accumulates FP16 products in FP32 only, so
  its FP16-accumulate ceiling equals the FP32-accumulate one (Ada's is twice).
  ``RTX4060_PROFILE`` is the reference's own audited profile.
- ``measure_peaks`` calibrates on the GPU: the best device-copy bandwidth (PyTorch's
  copy and the library's ``tk_roof_copy``), a hipBLASLt ``torch.mm`` FP16 sweep with
  the engine clock sampled by ``rocm-smi`` while it runs, and the theoretical ceiling
  at the highest clock observed. ``load_or_measure_peaks`` caches the result as JSON
  and reuses it only when ``_validate_stored_peaks`` accepts its provenance.
- The payload keeps the reference's field names so caches and tests carry over; on
  this build ``triton_version`` identifies the kernel library that produced the
  kernels (there is no Triton) and ``compute_capability`` is PyTorch's
  ``major.minor`` for the GPU (9.5 for gfx950).
"""

from __future__ import annotations

import datetime as _dt
import math
import re
import subprocess
import threading
import time
from collections.abc import Callable
from dataclasses import dataclass
from pathlib import Path
from typing import Generic, TypedDict, TypeVar, cast

import torch

from tklab.harness.jsonio import JsonObject, read_json_object, write_json_atomic
from tklab.harness.timing import time_ms

PEAKS_SCHEMA_VERSION = 7
DEFAULT_BW_ELEMENT_COUNTS = tuple(2**exponent for exponent in range(26, 29))
DEFAULT_TFLOPS_SIZES = (1024, 2048, 4096, 8192)
_UTILIZATION_LIMIT_PCT = 10
_AMD_MI355X_SPEC_URL = "https://www.amd.com/en/products/accelerators/instinct/mi350/mi355x.html"
_AMD_CDNA4_WHITEPAPER_URL = (
    "https://www.amd.com/content/dam/amd/en/documents/instinct-tech-docs/white-papers/"
    "amd-cdna-4-architecture-whitepaper.pdf"
)
_NVIDIA_RTX4060_SPEC_URL = (
    "https://www.nvidia.com/en-us/geforce/graphics-cards/40-series/rtx-4060-4060ti/"
)
_NVIDIA_ADA_WHITEPAPER_URL = (
    "https://images.nvidia.com/aem-dam/Solutions/geforce/ada/nvidia-ada-gpu-architecture.pdf"
)


@dataclass(frozen=True, slots=True)
class GpuTheoreticalProfile:
    """Hardware facts behind a clock-scaled dense FP16 matrix ceiling."""

    model_substring: str
    rated_boost_mhz: int
    streaming_multiprocessors: int
    tensor_cores_per_sm: int
    fp16_fp32acc_flops_per_clock_per_tensor_core: int
    product_spec_url: str
    architecture_whitepaper_url: str
    fp16acc_ratio: float = 1.0  # FP16-accumulate over FP32-accumulate throughput
    # Architecture name that identifies the GPU when its marketing name does not
    # (ROCm PyTorch reports gfx950 boards as "AMD Radeon Graphics").
    arch_substring: str = ""

    def fp16_fp32acc_tflops(self, clock_mhz: int) -> float:
        """Dense FP16-input / FP32-accumulate TFLOP/s at ``clock_mhz``."""
        return (
            self.streaming_multiprocessors
            * self.tensor_cores_per_sm
            * self.fp16_fp32acc_flops_per_clock_per_tensor_core
            * clock_mhz
            / 1e6
        )

    def fp16_fp16acc_tflops(self, clock_mhz: int) -> float:
        """Dense FP16-input / FP16-accumulate TFLOP/s at ``clock_mhz``."""
        return self.fp16acc_ratio * self.fp16_fp32acc_tflops(clock_mhz)


MI355X_PROFILE = GpuTheoreticalProfile(
    model_substring="MI355X",
    rated_boost_mhz=2400,
    streaming_multiprocessors=256,
    tensor_cores_per_sm=4,
    fp16_fp32acc_flops_per_clock_per_tensor_core=1024,
    product_spec_url=_AMD_MI355X_SPEC_URL,
    architecture_whitepaper_url=_AMD_CDNA4_WHITEPAPER_URL,
    fp16acc_ratio=1.0,
    arch_substring="gfx950",
)
RTX4060_PROFILE = GpuTheoreticalProfile(
    model_substring="RTX 4060",
    rated_boost_mhz=2460,
    streaming_multiprocessors=24,
    tensor_cores_per_sm=4,
    fp16_fp32acc_flops_per_clock_per_tensor_core=128,
    product_spec_url=_NVIDIA_RTX4060_SPEC_URL,
    architecture_whitepaper_url=_NVIDIA_ADA_WHITEPAPER_URL,
    fp16acc_ratio=2.0,
)
_GPU_PROFILES = (MI355X_PROFILE, RTX4060_PROFILE)
_ResultT = TypeVar("_ResultT")


class BandwidthSample(TypedDict):
    """One device-copy bandwidth observation."""

    elements: int
    working_set_bytes: int
    ms: float
    gbps: float


class TflopsSample(TypedDict):
    """One square GEMM throughput and engine-clock observation."""

    n: int
    ms: float
    tflops: float
    sm_clock_mhz: int
    sm_clock_min_mhz: int
    sm_clock_max_mhz: int
    sm_clock_samples_mhz: list[int]


class TheoreticalProvenance(TypedDict):
    """Serialized provenance of the theoretical compute ceilings."""

    model: str
    rated_boost_clock_mhz: int
    streaming_multiprocessors: int
    tensor_cores_per_sm: int
    fp16_fp32acc_flops_per_clock_per_tensor_core: int
    fp16_fp32acc_rated_tflops: float
    fp16_fp16acc_rated_tflops: float
    ceiling_clock_policy: str
    product_spec_url: str
    architecture_whitepaper_url: str


class PeakResults(TypedDict):
    """Versioned roofline-calibration payload."""

    schema_version: int
    gpu_name: str
    gpu_slug: str
    compute_capability: str
    torch_version: str
    triton_version: str
    calibration_started_at_utc: str
    calibration_preflight_gpu_utilization_pct: list[int]
    calibration_preflight_gpu_utilization_limit_pct: int
    peak_bw_gbps: float
    bandwidth_elements: int
    bandwidth_samples: list[BandwidthSample]
    cublas_tflops_fp16_fp32acc: float
    torch_fp16acc_available: bool
    theoretical_tflops_fp16_fp32acc_rated: float
    theoretical_tflops_fp16_fp32acc_at_measured_clock: float
    theoretical_tflops_fp16_fp16acc_rated: float
    theoretical_tflops_fp16_fp16acc_at_measured_clock: float
    theoretical_ceiling_sm_clock_mhz: int
    tflops_samples: list[TflopsSample]
    best_tflops_size: int
    best_tflops_sm_clock_mhz: int
    theoretical_provenance: TheoreticalProvenance


def torch_fp16acc_available() -> bool:
    """Whether this PyTorch exposes the FP16-accumulate GEMM switch (a version probe)."""
    return hasattr(torch.backends.cuda.matmul, "allow_fp16_accumulation")


def kernel_library_version() -> str:
    """Identity of the kernel library (stored as the payload's ``triton_version``)."""
    from tklab import _hip

    return f"tklab_hip abi {_hip.load_library().tk_abi_version()}"


def gpu_slug(device: int = 0) -> str:
    """Filesystem-safe slug of the GPU's name.

    Raises:
        RuntimeError: If no GPU or ``device`` is unavailable.
    """
    _validate_cuda_device(device)
    return re.sub(r"[^a-z0-9]+", "_", torch.cuda.get_device_name(device).lower()).strip("_")


def gpu_utilization_pct(device: int = 0) -> int:
    """Whole-device utilization in percent, from ``rocm-smi --showuse``.

    Raises:
        RuntimeError: If ``rocm-smi`` cannot provide the value.
    """
    return _rocm_smi_integer(
        ["--showuse"], r"GPU use \(%\)\s*:\s*(\d+)", device,
        "unable to query GPU utilization with rocm-smi",
    )


def _idle_utilization_samples(device: int, count: int = 5, timeout_s: float = 5.0) -> list[int]:
    """``count`` consecutive utilization samples at or below the limit. rocm-smi's
    figure is a trailing average, so work that just finished decays over a few
    samples; sampling continues for up to ``timeout_s``.

    Raises:
        RuntimeError: If the GPU stays busy.
    """
    samples: list[int] = []
    deadline = time.monotonic() + timeout_s
    while True:
        samples.append(gpu_utilization_pct(device))
        recent = samples[-count:]
        if len(recent) == count and max(recent) <= _UTILIZATION_LIMIT_PCT:
            return recent
        if time.monotonic() > deadline:
            raise RuntimeError(
                f"GPU {device} is busy ({recent} % use); calibrate on an idle GPU"
            )
        time.sleep(0.1)


def measured_peak_bw_gbps(
    device: int = 0,
    *,
    element_counts: tuple[int, ...] = DEFAULT_BW_ELEMENT_COUNTS,
    warmup_ms: int = 100,
    repetition_ms: int = 500,
) -> float:
    """Best sustained device-copy bandwidth in GB/s (one read plus one write)."""
    samples = _measure_bandwidth_samples(
        device, element_counts=element_counts, warmup_ms=warmup_ms, repetition_ms=repetition_ms
    )
    return max(sample["gbps"] for sample in samples)


def theoretical_tflops_fp16_fp32acc(
    sm_clock_mhz: int, *, profile: GpuTheoreticalProfile = MI355X_PROFILE
) -> float:
    """Theoretical dense FP16 / FP32-accumulate ceiling at ``sm_clock_mhz``."""
    return profile.fp16_fp32acc_tflops(sm_clock_mhz)


def theoretical_tflops_fp16_fp16acc(
    sm_clock_mhz: int, *, profile: GpuTheoreticalProfile = MI355X_PROFILE
) -> float:
    """Theoretical dense FP16 / FP16-accumulate ceiling at ``sm_clock_mhz``."""
    return profile.fp16_fp16acc_tflops(sm_clock_mhz)


def measure_peaks(
    device: int = 0,
    *,
    bw_element_counts: tuple[int, ...] = DEFAULT_BW_ELEMENT_COUNTS,
    tflops_sizes: tuple[int, ...] = DEFAULT_TFLOPS_SIZES,
    warmup_ms: int = 100,
    repetition_ms: int = 500,
) -> PeakResults:
    """Calibrate the roofs on ``device`` (reference ``roofline.py:240-351``).

    Raises:
        RuntimeError: If the GPU is busy before calibration or unavailable.
        ValueError: If the GPU has no audited profile.
    """
    _validate_cuda_device(device)
    name = torch.cuda.get_device_name(device)
    profile = _profile_for(name, _arch_name(device))
    started = _dt.datetime.now(_dt.timezone.utc).isoformat()
    utilization = _idle_utilization_samples(device)
    bandwidth = _measure_bandwidth_samples(
        device, element_counts=bw_element_counts, warmup_ms=warmup_ms, repetition_ms=repetition_ms
    )
    best_bw = max(bandwidth, key=lambda sample: sample["gbps"])
    tflops = _measure_tflops_samples(device, sizes=tflops_sizes, repetition_ms=repetition_ms)
    best = max(tflops, key=lambda sample: sample["tflops"])
    ceiling_clock = _maximum_observed_sm_clock_mhz(tflops)
    major, minor = torch.cuda.get_device_capability(device)
    provenance: TheoreticalProvenance = {
        "model": name,
        "rated_boost_clock_mhz": profile.rated_boost_mhz,
        "streaming_multiprocessors": profile.streaming_multiprocessors,
        "tensor_cores_per_sm": profile.tensor_cores_per_sm,
        "fp16_fp32acc_flops_per_clock_per_tensor_core":
            profile.fp16_fp32acc_flops_per_clock_per_tensor_core,
        "fp16_fp32acc_rated_tflops": profile.fp16_fp32acc_tflops(profile.rated_boost_mhz),
        "fp16_fp16acc_rated_tflops": profile.fp16_fp16acc_tflops(profile.rated_boost_mhz),
        "ceiling_clock_policy": "maximum observed clock",
        "product_spec_url": profile.product_spec_url,
        "architecture_whitepaper_url": profile.architecture_whitepaper_url,
    }
    return {
        "schema_version": PEAKS_SCHEMA_VERSION,
        "gpu_name": name,
        "gpu_slug": gpu_slug(device),
        "compute_capability": f"{major}.{minor}",
        "torch_version": torch.__version__,
        "triton_version": kernel_library_version(),
        "calibration_started_at_utc": started,
        "calibration_preflight_gpu_utilization_pct": utilization,
        "calibration_preflight_gpu_utilization_limit_pct": _UTILIZATION_LIMIT_PCT,
        "peak_bw_gbps": best_bw["gbps"],
        "bandwidth_elements": best_bw["elements"],
        "bandwidth_samples": bandwidth,
        "cublas_tflops_fp16_fp32acc": best["tflops"],
        "torch_fp16acc_available": torch_fp16acc_available(),
        "theoretical_tflops_fp16_fp32acc_rated": provenance["fp16_fp32acc_rated_tflops"],
        "theoretical_tflops_fp16_fp32acc_at_measured_clock":
            profile.fp16_fp32acc_tflops(ceiling_clock),
        "theoretical_tflops_fp16_fp16acc_rated": provenance["fp16_fp16acc_rated_tflops"],
        "theoretical_tflops_fp16_fp16acc_at_measured_clock":
            profile.fp16_fp16acc_tflops(ceiling_clock),
        "theoretical_ceiling_sm_clock_mhz": ceiling_clock,
        "tflops_samples": tflops,
        "best_tflops_size": best["n"],
        "best_tflops_sm_clock_mhz": best["sm_clock_mhz"],
        "theoretical_provenance": provenance,
    }


def load_or_measure_peaks(path: Path, device: int = 0, *, force: bool = False) -> PeakResults:
    """Reuse the cached calibration at ``path`` when its provenance matches this GPU and
    software, else measure and cache (reference ``roofline.py:354-405``)."""
    path = Path(path)
    if path.is_file() and not force:
        payload = read_json_object(path)
        major, minor = torch.cuda.get_device_capability(device)
        _validate_stored_peaks(
            payload,
            path=path,
            expected_gpu_name=torch.cuda.get_device_name(device),
            expected_compute_capability=f"{major}.{minor}",
            expected_torch_version=torch.__version__,
            expected_triton_version=kernel_library_version(),
        )
        return cast(PeakResults, payload)
    peaks = measure_peaks(device)
    write_json_atomic(path, cast(JsonObject, peaks))
    return peaks


def _measure_bandwidth_samples(
    device: int, *, element_counts: tuple[int, ...], warmup_ms: int, repetition_ms: int
) -> list[BandwidthSample]:
    """Copy bandwidth per working set: the better of PyTorch's device copy and
    ``tk_roof_copy`` (16-byte non-temporal streaming), counting a read and a write."""
    from tklab import _hip

    samples: list[BandwidthSample] = []
    dev = torch.device("cuda", device)
    for elements in element_counts:
        src = torch.ones(elements, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        nbytes = elements * 4
        stream = _hip.stream_of(src)
        candidates = [
            lambda: dst.copy_(src),
            lambda: _hip.call("tk_roof_copy", src.data_ptr(), dst.data_ptr(), nbytes, stream),
        ]
        ms = min(
            cast(float, time_ms(fn, warmup_ms=warmup_ms, repetition_ms=repetition_ms, device=dev))
            for fn in candidates
        )
        if not torch.equal(src, dst):
            raise RuntimeError("device copy produced a wrong result during calibration")
        samples.append({"elements": elements, "working_set_bytes": 2 * nbytes, "ms": ms,
                        "gbps": 2 * nbytes / ms / 1e6})
        del src, dst
    return samples


def _maximum_observed_sm_clock_mhz(*sample_groups: list[TflopsSample]) -> int:
    """Highest engine clock sampled across the compute calibration sweeps
    (reference ``roofline.py:444-455``).

    Raises:
        ValueError: If no compute samples are supplied.
    """
    clocks = [sample["sm_clock_max_mhz"] for group in sample_groups for sample in group]
    if not clocks:
        raise ValueError("at least one compute clock sample is required")
    return max(clocks)


def _measure_tflops_samples(
    device: int, *, sizes: tuple[int, ...], repetition_ms: int
) -> list[TflopsSample]:
    """hipBLASLt FP16 ``torch.mm`` throughput per size, warmed to a steady clock, with
    the engine clock sampled while the timed launches run."""
    dev = torch.device("cuda", device)
    samples: list[TflopsSample] = []
    for n in sizes:
        a = torch.randn(n, n, device=dev, dtype=torch.float16) * n ** -0.25
        b = torch.randn(n, n, device=dev, dtype=torch.float16) * n ** -0.25
        c = torch.empty(n, n, device=dev, dtype=torch.float16)
        call = lambda: torch.mm(a, b, out=c)  # noqa: E731
        _warm_to_steady_clock(call)
        monitored = _measure_with_clock_monitor(
            lambda: cast(float, time_ms(call, warmup_ms=25, repetition_ms=repetition_ms,
                                        device=dev)),
            device,
        )
        clocks = monitored.clock_samples_mhz
        samples.append({
            "n": n,
            "ms": monitored.value,
            "tflops": 2 * n**3 / monitored.value / 1e9,
            "sm_clock_mhz": int(round(sum(clocks) / len(clocks))),
            "sm_clock_min_mhz": min(clocks),
            "sm_clock_max_mhz": max(clocks),
            "sm_clock_samples_mhz": clocks,
        })
        del a, b, c
    return samples


@dataclass(frozen=True, slots=True)
class _MonitoredResult(Generic[_ResultT]):
    value: _ResultT
    clock_samples_mhz: list[int]


def _measure_with_clock_monitor(
    fn: Callable[[], _ResultT], device: int, interval_s: float = 0.05
) -> _MonitoredResult[_ResultT]:
    """Run ``fn`` while a thread samples the engine clock; at least one sample is taken
    after ``fn`` returns if the run was shorter than one query."""
    samples: list[int] = []
    stop = threading.Event()

    def poll() -> None:
        while not stop.is_set():
            try:
                samples.append(_sm_clock_mhz(device))
            except RuntimeError:
                return
            stop.wait(interval_s)

    thread = threading.Thread(target=poll, daemon=True)
    thread.start()
    try:
        value = fn()
    finally:
        stop.set()
        thread.join()
    if not samples:
        samples.append(_sm_clock_mhz(device))
    return _MonitoredResult(value, samples)


def _warm_to_steady_clock(fn: Callable[[], object], seconds: float = 3.0) -> None:
    """Launch ``fn`` back to back for ``seconds`` so the clock settles under load."""
    deadline = time.perf_counter() + seconds
    while time.perf_counter() < deadline:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def _sm_clock_mhz(device: int = 0) -> int:
    """Current engine (shader) clock in MHz, from the ``sclk`` line of
    ``rocm-smi --showclocks`` (its level field is a number or ``S``)."""
    return _rocm_smi_integer(
        ["--showclocks"], r"sclk clock level:\s*\S+:\s*\((\d+)\s*[Mm][Hh]z\)", device,
        "unable to query the engine clock with rocm-smi",
    )


def _rocm_smi_integer(args: list[str], pattern: str, device: int, error_message: str) -> int:
    """First integer captured by ``pattern`` in ``rocm-smi -d device <args>``.

    Raises:
        RuntimeError: If the tool is missing, fails, or prints no match.
    """
    try:
        out = subprocess.run(
            ["rocm-smi", "-d", str(device), *args],
            check=True, capture_output=True, text=True, timeout=10,
        ).stdout
        match = re.search(pattern, out)
        if match is None:
            raise ValueError(out[-200:])
        return int(match.group(1))
    except (FileNotFoundError, subprocess.CalledProcessError, subprocess.TimeoutExpired,
            ValueError) as error:
        raise RuntimeError(error_message) from error


def _profile_for(gpu_name: str, arch_name: str = "") -> GpuTheoreticalProfile:
    """Audited profile matching ``gpu_name`` or, failing that, ``arch_name`` (the
    device's ``gcnArchName``). gfx950 maps to the MI355X profile, the one audited
    gfx950 part here.

    Raises:
        ValueError: If the GPU has no audited profile.
    """
    for profile in _GPU_PROFILES:
        if profile.model_substring in gpu_name:
            return profile
    for profile in _GPU_PROFILES:
        if profile.arch_substring and profile.arch_substring in arch_name:
            return profile
    raise ValueError(
        f"no theoretical compute profile for {gpu_name!r}; "
        "add an audited GpuTheoreticalProfile before benchmarking compute kernels"
    )


def _arch_name(device: int) -> str:
    """The device's ``gcnArchName`` ("" where PyTorch does not report one)."""
    return str(getattr(torch.cuda.get_device_properties(device), "gcnArchName", ""))


def _validate_cuda_device(device: int) -> None:
    """Validate that GPU ``device`` can be selected."""
    if device < 0:
        raise ValueError("device index must be non-negative")
    if not torch.cuda.is_available():
        raise RuntimeError("no GPU (ROCm/HIP) is available")
    if device >= torch.cuda.device_count():
        raise RuntimeError(
            f"GPU device {device} is unavailable; found {torch.cuda.device_count()} device(s)"
        )


_REQUIRED_FIELDS = frozenset({
    "gpu_name",
    "peak_bw_gbps",
    "cublas_tflops_fp16_fp32acc",
    "theoretical_tflops_fp16_fp32acc_at_measured_clock",
    "theoretical_tflops_fp16_fp16acc_at_measured_clock",
    "theoretical_ceiling_sm_clock_mhz",
    "theoretical_provenance",
    "calibration_started_at_utc",
    "calibration_preflight_gpu_utilization_pct",
    "calibration_preflight_gpu_utilization_limit_pct",
})
_POSITIVE_FIELDS = (
    "cublas_tflops_fp16_fp32acc",
    "peak_bw_gbps",
    "theoretical_ceiling_sm_clock_mhz",
    "theoretical_tflops_fp16_fp16acc_at_measured_clock",
    "theoretical_tflops_fp16_fp32acc_at_measured_clock",
)
_PROVENANCE_FIELDS = frozenset(TheoreticalProvenance.__annotations__)


def _is_percent(value: object) -> bool:
    return isinstance(value, int) and not isinstance(value, bool) and 0 <= value <= 100


def _validate_stored_peaks(
    payload: JsonObject,
    *,
    path: Path,
    expected_gpu_name: str,
    expected_compute_capability: str,
    expected_torch_version: str,
    expected_triton_version: str,
) -> None:
    """Validate a cached calibration against the active GPU and software
    (reference ``roofline.py:636-745``): schema version, required fields, the
    preflight utilization samples and limit, finite positive roofs, a complete
    theoretical provenance, then GPU name, compute capability, PyTorch version and
    kernel-library version.

    Raises:
        ValueError: On the first check that fails, naming ``path``.
    """
    if payload.get("schema_version") != PEAKS_SCHEMA_VERSION:
        raise ValueError(f"{path}: incompatible peaks schema; rerun with --force-peaks")
    missing = sorted(_REQUIRED_FIELDS.difference(payload))
    if missing:
        raise ValueError(f"{path}: missing required fields: {', '.join(missing)}")
    samples = payload["calibration_preflight_gpu_utilization_pct"]
    if not isinstance(samples, list) or not samples or not all(map(_is_percent, samples)):
        raise ValueError(f"{path}: invalid calibration GPU-utilization samples")
    limit = payload["calibration_preflight_gpu_utilization_limit_pct"]
    if not _is_percent(limit) or max(samples) > limit:
        raise ValueError(f"{path}: invalid calibration GPU-utilization limit")
    invalid = [
        name for name in _POSITIVE_FIELDS
        if not isinstance(payload[name], int | float) or isinstance(payload[name], bool)
        or not math.isfinite(payload[name]) or payload[name] <= 0
    ]
    if invalid:
        raise ValueError(
            f"{path}: cached peaks contain invalid positive numeric fields: {', '.join(invalid)}"
        )
    provenance = payload["theoretical_provenance"]
    if not isinstance(provenance, dict):
        raise ValueError(f"{path}: theoretical_provenance must be an object")
    missing = sorted(_PROVENANCE_FIELDS.difference(provenance))
    if missing:
        raise ValueError(
            f"{path}: theoretical_provenance is missing fields: {', '.join(missing)}"
        )
    expected = {
        "gpu_name": expected_gpu_name,
        "compute_capability": expected_compute_capability,
        "torch_version": expected_torch_version,
        "triton_version": expected_triton_version,
    }
    mismatches = [
        f"{field}={payload.get(field)!r} (expected {value!r})"
        for field, value in expected.items()
        if payload.get(field) != value
    ]
    if mismatches:
        raise ValueError(
            f"{path}: cached peaks do not match the active environment: "
            f"{'; '.join(mismatches)}; rerun with --force-peaks"
        )
