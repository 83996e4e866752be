#!/usr/bin/env python3
"""Benchmark of the MI355X tklab kernels; prints one JSON line.

Step (the timed unit): benchmark config 2 — residual RMSNorm forward + backward
on bfloat16 x, residual [16384, 4096] (weight ~ N(1, 0.02), eps 1e-6, both
upstream gradients ~ N(0, 1)), i.e. three launches into preallocated buffers:
tk_rmsnorm_fwd (with residual), tk_rmsnorm_bwd_stage1 (with the incoming sum
gradient) and tk_rmsnorm_bwd_stage2. Algorithmic bytes per step:
forward 4*M*D*2 + backward 4*M*D*2 = 1 073 741 824 (weight, rstd and the
float32 partial rows are not counted).

``value`` is that step's throughput in GB/s with inputs resident in HBM; the steps
rotate over three independent tensor sets (STEP_SETS), so no step finds its tensors
in the last-level cache from the step before.
``roofline`` prices the dominant kernel of the step against 8 TB/s: its
algorithmic bytes per launch over its average duration, measured with one event
pair on the launch stream around K back-to-back launches of that kernel over the
step's tensor sets, after the timed steps (an untimed attribution pass with events
around every launch picks it; `attribution_ms`). ``traffic`` comes from the
committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary when present.
``reference_gpu`` times the reference's PyTorch path for the same step on the GPU.
``cpu_baseline`` times that PyTorch path on the host CPU (float32 upcasts, full size);
``cpu_oracle_port`` the CPU oracle (oracle/tklab_oracle.c) on a row sample.
``kernels`` times every other benchmark configuration (softmax, SwiGLU, RoPE,
GEMM, attention) per kernel, each beside torch's own GPU path for the same work
(``reference_ms``, ``speedup``). Memory-bound rows run back-to-back launches that
rotate over enough copies of their tensors to touch at least 1 GiB (four times
the 256 MiB last-level cache), so they measure steady HBM streaming without
cache reuse; MFMA rows flush 1 GiB before each launch.
``measured_roofs`` holds the ceilings this GPU sustains (the library's copy and
dense-MFMA calibration kernels, the HBM read:write mixes with the better of two store
policies); every row and ``roofline`` also carry
``frac_measured`` against them, beside ``frac`` against the published peaks. The
softmax row, a launch of ~23 us, also carries the stream roof of its own read:write mix
at its own bytes per launch (``matched_roof_GBps``, ``frac_matched``): launches that
short pay a dispatch ramp and last-wave drain of ~1-2 us that the large-array roofs
amortize.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-kernels] [--no-cpu] [--only TEXT]
"""

from __future__ import annotations

import argparse
import itertools
import json
import math
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "triton-kernel-lab_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "% of roofline: HBM GB/s (norm/softmax) + TFLOP/s (GEMM, causal FA fwd+bwd)"
HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = {"float16": 2500.0, "bfloat16": 2500.0}
ROWS, COLS = 16384, 4096
EPS = 1e-6
TRAFFIC_SUMMARY = ROOT / "profiles" / "rmsnorm_bwd_stage1_traffic.txt"


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-kernels", action="store_true", help="skip the per-config kernel table")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", default=None,
                   help="time only the kernel-table rows whose kernel name or config contains "
                        "this text (for profiling one kernel family or one shape)")
    return p.parse_args()


def progress(message: str) -> None:
    """One line on stderr per finished phase or row (stdout carries only the JSON line)."""
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def _traffic_from_summary() -> float | None:
    """HBM bytes per stage-1 launch from the committed rocprofv3 PMC summary."""
    if not TRAFFIC_SUMMARY.is_file():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", TRAFFIC_SUMMARY.read_text(), re.M)
    return float(m.group(1)) if m else None


# Independent input/output sets the steps rotate over: step i uses set i % STEP_SETS, so
# no step finds its tensors in the 256 MiB last-level cache from the step before (one set
# of seven 128 MiB tensors is only 3.5 times that cache; a single reused set ran the step
# ~5 % faster).
STEP_SETS = 3


class StepSet:
    """One set of the step's preallocated tensors (set 0 is seeded like the CPU baseline)."""

    def __init__(self, torch, device, rn, g) -> None:
        bf16 = torch.bfloat16
        self.x = torch.randn(ROWS, COLS, device=device, dtype=bf16, generator=g)
        self.r = torch.randn(ROWS, COLS, device=device, dtype=bf16, generator=g)
        self.w = (1 + 0.02 * torch.randn(COLS, device=device, generator=g)).to(bf16)
        self.dsum = torch.randn(ROWS, COLS, device=device, dtype=bf16, generator=g)
        self.dout = torch.randn(ROWS, COLS, device=device, dtype=bf16, generator=g)
        self.s = torch.empty_like(self.x)
        self.y = torch.empty_like(self.x)
        self.rstd = torch.empty(ROWS, device=device, dtype=torch.float32)
        self.buffers = rn._make_backward_buffers(self.s, self.w)


class Step:
    """Preallocated buffers and the three launches of one residual-RMSNorm fwd+bwd step,
    over STEP_SETS independent tensor sets."""

    def __init__(self, torch, device, sets: int = STEP_SETS) -> None:
        from tklab.kernels import residual_rms_norm as rrn
        from tklab.kernels import rms_norm as rn

        self.rrn, self.rn = rrn, rn
        g = torch.Generator(device=device).manual_seed(0)
        self.sets = [StepSet(torch, device, rn, g) for _ in range(sets)]

    def launches(self, i: int = 0):
        """The launches of step i (tensor set i % STEP_SETS)."""
        t = self.sets[i % len(self.sets)]
        b = t.buffers
        return (
            ("tk_rmsnorm_fwd", lambda: self.rrn._launch_forward(
                t.x, t.r, t.w, t.s, t.y, t.rstd,
                eps=EPS, store_residual=True, store_stats=True)),
            ("tk_rmsnorm_bwd_stage1", lambda: self.rn._launch_backward_stage1(
                t.dout, t.s, t.w, t.rstd, b, incoming_dx=t.dsum)),
            ("tk_rmsnorm_bwd_stage2", lambda: self.rn._launch_backward_stage2(b, COLS)),
        )


# Algorithmic bytes per launch (4 bf16 matrices each for forward and stage 1).
STEP_BYTES = {
    "tk_rmsnorm_fwd": 4 * ROWS * COLS * 2,
    "tk_rmsnorm_bwd_stage1": 4 * ROWS * COLS * 2,
    "tk_rmsnorm_bwd_stage2": 0,
}


def time_step(torch, step: Step, steps: int, warmup: int) -> tuple[float, str, float, dict]:
    """W untimed steps, an untimed attribution pass, K timed steps, then the dominant
    kernel on its own.

    The attribution pass (20 steps, events around every launch) gives each kernel's mean
    duration and picks the dominant one. The K timed steps carry no event but the pair
    around all of them: an event recorded between two dependent launches delays the
    second by several microseconds (events around every launch made the step ~8 % slower,
    and an event pair around one ~90 us kernel read it ~7 % long against the kernel
    trace). The dominant kernel's duration is then timed the same way: K launches back
    to back over the STEP_SETS tensor sets between one event pair, on the launch stream.
    Returns (ms per timed step, dominant kernel, its ms per launch, attribution-pass ms
    per kernel).
    """
    plans = [step.launches(i) for i in range(len(step.sets))]
    launches = plans[0]
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        for _, fn in plans[i % len(plans)]:
            fn()
    torch.cuda.synchronize()
    probe = 20
    pairs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in launches] for _ in range(probe)]
    for i in range(probe):
        for j, (_, fn) in enumerate(plans[i % len(plans)]):
            pairs[i][j][0].record(stream)
            fn()
            pairs[i][j][1].record(stream)
    torch.cuda.synchronize()
    attribution = {name: statistics.fmean(pairs[i][j][0].elapsed_time(pairs[i][j][1])
                                          for i in range(probe))
                   for j, (name, _) in enumerate(launches)}
    dominant = max(attribution, key=attribution.get)
    dom = [name for name, _ in launches].index(dominant)

    def timed_region(body) -> tuple[float, float]:
        """(event ms, host ms) around `steps` calls of body(i) on the launch stream."""
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record(stream)
        for i in range(steps):
            body(i)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end), (time.perf_counter() - t0) * 1e3

    def one_step(i):
        for _, fn in plans[i % len(plans)]:
            fn()

    event_ms, wall_ms = timed_region(one_step)
    ms_step = event_ms / steps
    # The event clock and the host clock must agree on the timed region.
    if abs(wall_ms / steps - ms_step) > 0.5 * ms_step:
        raise RuntimeError(f"event and host clocks disagree: {ms_step} vs {wall_ms / steps} ms")
    dominant_ms = timed_region(lambda i: plans[i % len(plans)][dom][1]())[0] / steps
    return ms_step, dominant, dominant_ms, attribution


def _cpu_facts() -> dict:
    """Host CPU model, logical CPUs, physical cores and the CPUs this process may use."""
    model, cores = None, set()
    try:
        phys = core = None
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name" and model is None:
                model = val
            elif key == "physical id":
                phys = val
            elif key == "core id":
                core = val
            elif not key and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(),
            "physical_cores": len(cores) or None, "usable_cpus": usable}


def torch_gpu_step_ms(torch, step: Step, steps: int) -> float:
    """The reference's PyTorch path for the step on the GPU in the step's dtype: x + r,
    F.rms_norm and torch.autograd.grad of both outputs (what the reference's benchmark
    times beside its kernels), rotating over the step's tensor sets like the timed steps.
    Mean ms per step over `steps` after 3 warmups."""
    import torch.nn.functional as F

    sets = [([t.x.detach().requires_grad_(True), t.r.detach().requires_grad_(True),
              t.w.detach().requires_grad_(True)], (t.dsum, t.dout)) for t in step.sets]

    def once(i):
        leaves, grads = sets[i % len(sets)]
        s_ = leaves[0] + leaves[1]
        y_ = F.rms_norm(s_, (COLS,), leaves[2], EPS)
        return torch.autograd.grad((s_, y_), leaves, grads)

    for i in range(3):
        once(i)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    for i in range(steps):
        once(i)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def cpu_baseline(torch, reps: int = 5) -> dict:
    """The reference's own PyTorch path for the step on the host CPU.

    The reference checks its kernels against ``x + r`` -> ``F.rms_norm`` and
    ``torch.autograd.grad`` evaluated on float32 upcasts (its ``ref_fn``,
    ``residual_rms_norm.py:279-286``, and ``tests/test_correctness.py:40``). This times
    exactly that on the full 16384 x 4096 workload (same seeded draws as the GPU step,
    rounded to bf16, then upcast), one warmup and the median of `reps`, and reports it
    with the step's algorithmic byte count. Threads: the physical cores this process may
    use, capped at 16 (the CPU share of one GPU on the benchmark boxes). A native-bf16
    run of the same path is reported beside it.
    """
    import torch.nn.functional as F

    facts = _cpu_facts()
    usable = facts["usable_cpus"] or 1
    threads = max(1, min(16, facts["physical_cores"] or usable, usable))
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        g = torch.Generator().manual_seed(0)
        bf16 = torch.bfloat16
        x = torch.randn(ROWS, COLS, generator=g).to(bf16)
        r = torch.randn(ROWS, COLS, generator=g).to(bf16)
        w = (1 + 0.02 * torch.randn(COLS, generator=g)).to(bf16)
        dsum = torch.randn(ROWS, COLS, generator=g).to(bf16)
        dout = torch.randn(ROWS, COLS, generator=g).to(bf16)

        def run(dtype) -> list[float]:
            leaves = [t.to(dtype).requires_grad_(True) for t in (x, r, w)]
            grads = (dsum.to(dtype), dout.to(dtype))
            times = []
            for _ in range(reps + 1):
                t0 = time.perf_counter_ns()
                s_ = leaves[0] + leaves[1]
                y_ = F.rms_norm(s_, (COLS,), leaves[2], EPS)
                torch.autograd.grad((s_, y_), leaves, grads)
                times.append((time.perf_counter_ns() - t0) / 1e9)
            return times[1:]

        f32 = run(torch.float32)
        native = run(bf16)
    finally:
        torch.set_num_threads(previous)
    step_bytes = sum(STEP_BYTES.values())
    med32, medbf = statistics.median(f32), statistics.median(native)
    return {
        "value": round(step_bytes / med32 / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "reference",
        "impl": "torch",
        "ms_per_step": round(med32 * 1e3, 2),
        "bf16_native_value": round(step_bytes / medbf / 1e9, 3),
        "bf16_native_ms_per_step": round(medbf * 1e3, 2),
        "torch_threads": threads,
        **facts,
        "sample": f"the reference's PyTorch path (x + r, F.rms_norm, torch.autograd.grad of both "
                  f"outputs) on float32 upcasts of the full {ROWS} x {COLS} step, median of "
                  f"{reps} after 1 warmup, {threads} torch threads; value uses the step's "
                  f"{step_bytes} algorithmic bytes",
    }


def cpu_oracle_port(seconds: float) -> dict:
    """The CPU oracle (C restatement) on a 2048-row sample, repeated for ~`seconds`."""
    import numpy as np

    from oracle import oracle

    threads = min(16, os.cpu_count() or 1)
    oracle.set_threads(threads)
    rng = np.random.default_rng(0)
    rows = 2048
    to_bf16 = lambda a: oracle.round_to(a.astype(np.float32), "bfloat16")  # noqa: E731
    x = to_bf16(rng.standard_normal((rows, COLS)))
    r = to_bf16(rng.standard_normal((rows, COLS)))
    w = to_bf16(1 + 0.02 * rng.standard_normal(COLS))
    dsum = to_bf16(rng.standard_normal((rows, COLS)))
    dout = to_bf16(rng.standard_normal((rows, COLS)))
    passes = 0
    t0 = time.perf_counter()
    while True:
        s, _, rstd = oracle.rmsnorm_fwd(x, w, EPS, "bfloat16", residual=r)
        oracle.rmsnorm_bwd(dout, s, w, rstd, "bfloat16", incoming=dsum)
        passes += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    sample_bytes = 8 * rows * COLS * 2
    return {
        "value": round(sample_bytes * passes / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle residual RMSNorm fwd+bwd, {rows} x {COLS} bf16-valued rows, "
                  f"{passes} passes in {elapsed:.1f} s (OpenMP, {threads} threads)",
    }


def measured_roofs(torch, device) -> dict:
    """Roofs this GPU sustains, from the library's calibration kernels.

    Copy: tk_roof_copy of 1 GiB back to back (2 GiB of HBM traffic per launch),
    beside torch's own device copy; the larger is the copy roof. MFMA: tk_roof_mfma
    with 8192 waves (8 per SIMD) of dense v_mfma_f32_16x16x32 (the shape that
    sustains the most FLOP/s under the power limit) and no memory traffic, timed like
    the MFMA rows (25 ms of warmup, then a 1 GiB flush before each launch), at about
    the length of the 8192^3 GEMM (~1 ms) and of the causal attention forward (~4 ms).
    """
    from tklab import _hip

    src = torch.ones(1 << 28, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    nbytes = src.numel() * 4
    stream = torch.cuda.current_stream().cuda_stream

    def copy_ms(fn, reps: int = 20) -> float:
        for _ in range(3):
            fn()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    own = 2 * nbytes / copy_ms(lambda: _hip.call("tk_roof_copy", src.data_ptr(), dst.data_ptr(),
                                                  nbytes, stream)) / 1e6
    ref = 2 * nbytes / copy_ms(lambda: dst.copy_(src)) / 1e6
    if not torch.equal(src, dst):
        raise RuntimeError("tk_roof_copy produced a wrong copy")
    del src, dst
    # Read:write mixes, each the best of two layouts (128 MiB per array, the step's tensor
    # size, rotating over three independent sets like the step; 512 MiB per array, one set)
    # and eight access variants: 8 or 16 KiB tiles, one workgroup per tile or 8192
    # workgroups walking them grid-stride, non-temporal or sc1 stores.
    big = 1 << 29
    srcs = torch.randint(-2**31, 2**31 - 1, (3 * big // 4,), dtype=torch.int32, device=device)
    dsts = torch.empty(2 * big // 4, dtype=torch.int32, device=device)
    mixes: dict[str, float] = {}
    policies: dict[str, str] = {}
    small = 1 << 27
    chunks = small // 16
    want = srcs[:3 * small // 4].view(3, chunks, 4)
    want = want[0] ^ want[1] ^ want[2]
    want[:, 0] ^= torch.arange(chunks, device=device, dtype=torch.int32)
    for reads, writes in ((1, 0), (0, 1), (1, 1), (2, 1), (3, 1), (2, 2), (3, 2)):
        key = f"{reads}:{writes}"
        for (part, nsets), policy, tile, grid in itertools.product(
                ((small, 3), (big, 1)), (0, 1), (8, 16), (0, 8192)):
            if writes == 0 and policy == 1:
                continue  # the store policy does not apply to a read-only stream
            turn = itertools.count()

            def launch(reads=reads, writes=writes, policy=policy, tile=tile, grid=grid,
                       part=part, nsets=nsets, turn=turn):
                k = next(turn) % nsets
                _hip.call("tk_roof_stream", srcs.data_ptr() + k * 3 * part,
                          dsts.data_ptr() + k * 2 * part, part, reads, writes, policy, tile,
                          grid, stream)

            ms = copy_ms(launch, reps=30)
            gbps = round((reads + writes) * part / ms / 1e6, 1)
            if gbps > mixes.get(key, 0.0):
                mixes[key] = gbps
                policies[key] = (f"{part >> 20} MiB x {nsets}, {tile} KiB tiles, "
                                 f"{'grid-stride' if grid else 'one per workgroup'}, "
                                 + (f"{('nt', 'sc1')[policy]} stores" if writes else "no stores"))
            if (reads, writes) == (3, 2) and part == small:
                got = dsts[:2 * small // 4].view(2, chunks, 4)
                if not (torch.equal(got[0], want) and torch.equal(got[1], want)):
                    raise RuntimeError("tk_roof_stream (3:2) produced wrong data")
                dsts.zero_()
    del srcs, dsts, want
    flush = torch.empty(1 << 28, dtype=torch.float32, device=device)
    waves = 8192
    out = torch.empty(waves, dtype=torch.float32, device=device)
    mfma: dict[str, dict[str, float]] = {}
    for dt_name, code in (("float16", 1), ("bfloat16", 2)):
        mfma[dt_name] = {}
        for label, iters in (("1ms", 1000), ("4ms", 4000)):
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < 0.025:
                _hip.call("tk_roof_mfma", code, out.data_ptr(), waves, iters, stream)
                torch.cuda.synchronize()
            times = []
            for _ in range(6):
                flush.zero_()
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record()
                _hip.call("tk_roof_mfma", code, out.data_ptr(), waves, iters, stream)
                b.record()
                times.append((a, b))
            torch.cuda.synchronize()
            ms = statistics.median(x.elapsed_time(y) for x, y in times[1:])
            mfma[dt_name][label] = round(waves * iters * 8 * 32768 / ms / 1e9, 1)
        if not bool(torch.isfinite(out).all()):
            raise RuntimeError("tk_roof_mfma produced non-finite sums")
    del flush, out
    torch.cuda.empty_cache()
    copy = max(own, ref)
    return {
        "hbm_GBps": round(max(copy, *mixes.values()), 1),
        "copy_GBps": round(copy, 1),
        "copy_kernels_GBps": {"tk_roof_copy": round(own, 1), "torch copy_": round(ref, 1)},
        "stream_mixes_GBps": mixes,
        "stream_mix_variant": policies,
        "mfma_TFLOPs": mfma,
        "note": "measured on this GPU by bench.py; frac_measured divides by hbm_GBps, the best "
                "of the copy and the tk_roof_stream read:write mixes (HBM rows), or by the MFMA "
                "roof of the nearer burst length (MFMA rows)",
    }


def kernel_table(torch, device, roofs: dict | None = None, only: str | None = None) -> list[dict]:
    """Per-kernel timings of every benchmark configuration (see the module docstring); with
    `only`, just the rows whose kernel name or config contains it."""
    from tklab.kernels import flash_attention as fa
    from tklab.kernels import fused_softmax as sm
    from tklab.kernels import matmul as mm
    from tklab.kernels import rope as rp
    from tklab.kernels import swiglu as sg

    flush = torch.empty(1 << 28, dtype=torch.float32, device=device)  # 1 GiB
    rows: list[dict] = []

    def timed(fn, reps: int) -> float:
        # The reference's timing (bench.py:98-103): at least 25 ms of warmup, then at
        # least 100 ms of timed launches; the median single launch.
        fn()
        torch.cuda.synchronize()
        t0, warm = time.perf_counter(), 0
        while time.perf_counter() - t0 < 0.025:
            fn()
            torch.cuda.synchronize()
            warm += 1
        each = (time.perf_counter() - t0) / max(warm, 1)
        reps = max(reps, math.ceil(0.1 / max(each, 1e-6)))
        times = []
        for _ in range(reps):
            flush.zero_()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            times.append((a, b))
        torch.cuda.synchronize()
        return statistics.median(x.elapsed_time(y) for x, y in times)

    def streamed(make, nbytes: int, reps: int) -> float:
        """Mean ms per launch, back to back, rotating over >= 1 GiB of tensor copies."""
        copies = max(1, -(-(1 << 30) // nbytes))
        fns = [make(i) for i in range(copies)]
        for fn in fns:
            fn()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for i in range(reps):
            fns[i % copies]()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    def add_reference(row, name, measure):
        """torch's own GPU path for the same work (the reference's ref_fn: eager PyTorch,
        hipBLASLt, SDPA), timed the same way as the row; `speedup` = reference_ms / ms."""
        if measure is None:
            return
        try:
            ref_ms = measure()
        except (RuntimeError, NotImplementedError) as exc:  # e.g. no SDPA backend for a shape
            row["reference"] = name
            row["reference_error"] = str(exc).splitlines()[0][:160]
            torch.cuda.synchronize()
            return
        row["reference"] = name
        row["reference_ms"] = round(ref_ms, 4)
        row["speedup"] = round(ref_ms / row["ms"], 3)

    def matched_roof(reads: int, writes: int, nbytes: int, reps: int) -> float:
        """Best tk_roof_stream rate for this read:write mix at exactly `nbytes` per launch
        (nbytes / (reads + writes) per array), back to back over the same number of rotating
        copies as the row, over the store policies, tile sizes and grid shapes of
        measured_roofs. A launch this short pays the dispatch ramp and the drain of its
        last wave, which the large-array roofs amortize."""
        from tklab import _hip

        part = nbytes // (reads + writes)
        copies = max(1, -(-(1 << 30) // nbytes))
        src = torch.empty(copies * reads * part // 4, dtype=torch.int32, device=device)
        dst = torch.empty(copies * writes * part // 4, dtype=torch.int32, device=device)
        stream = torch.cuda.current_stream().cuda_stream
        best = 0.0
        for policy, tile, grid in itertools.product((0, 1), (8, 16), (0, 8192)):
            def make(k, policy=policy, tile=tile, grid=grid):
                return lambda: _hip.call("tk_roof_stream", src.data_ptr() + k * reads * part,
                                         dst.data_ptr() + k * writes * part, part, reads, writes,
                                         policy, tile, grid, stream)
            best = max(best, nbytes / streamed(make, nbytes, reps) / 1e6)
        del src, dst
        return best

    def mem_row(name, config, make, nbytes, mix, reps=30, ref=None, ref_make=None, moved=1.0,
                size_matched=False):
        """`make(i)` returns the launch for tensor copy i (copy 0 may reuse the originals);
        `ref_make(i)` the torch reference's call on the same copy. `mix` is the kernel's
        read:write byte ratio, whose measured roof gives `frac_mix` for the bytes the kernel
        moves (`moved` times the algorithmic bytes). `size_matched`: also the stream roof of
        that mix at the row's own bytes per launch (`matched_roof_GBps`, `frac_matched`)."""
        if only and only not in name and only not in config:
            return False
        ms = streamed(make, nbytes, reps)
        gbps = nbytes / ms / 1e6
        row = {"kernel": name, "config": config, "ms": round(ms, 4), "bytes": nbytes,
               "GB/s": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4), "mix": mix}
        if roofs:
            row["frac_measured"] = round(gbps / roofs["hbm_GBps"], 4)
            row["frac_mix"] = round(moved * gbps / roofs["stream_mixes_GBps"][mix], 4)
            if size_matched:
                reads, writes = (int(v) for v in mix.split(":"))
                roof = matched_roof(reads, writes, int(moved * nbytes), reps)
                row["matched_roof_GBps"] = round(roof, 1)
                row["frac_matched"] = round(moved * gbps / roof, 4)
        if moved != 1.0:
            row["moved_GB/s"] = round(moved * gbps, 1)
        add_reference(row, ref, None if ref_make is None else
                      (lambda: streamed(ref_make, nbytes, reps)))
        rows.append(row)
        progress(f"{name} {config}: {row['ms']} ms")
        return True

    def mfma_row(name, config, fn, flops, dtype, reps=10, ref=None, ref_fn=None):
        if only and only not in name and only not in config:
            return False
        ms = timed(fn, reps)
        tf = flops / ms / 1e9
        row = {"kernel": name, "config": config, "ms": round(ms, 4), "flops": flops,
               "TFLOP/s": round(tf, 1), "frac": round(tf / MFMA_PEAK_TFLOPS[dtype], 4)}
        if roofs:
            roof = roofs["mfma_TFLOPs"][dtype]["1ms" if ms < 2.5 else "4ms"]
            row["frac_measured"] = round(tf / roof, 4)
        add_reference(row, ref, None if ref_fn is None else (lambda: timed(ref_fn(), reps)))
        rows.append(row)
        progress(f"{name} {config}: {row['ms']} ms")
        return True

    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    # SDPA references run on the fused backends only: the math backend issues bf16 batched
    # products on transposed views.
    fused_sdpa = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]

    def sdpa_fwd(q, k, v, causal, gqa=False):
        def go():
            with sdpa_kernel(fused_sdpa):
                return F.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=gqa)
        return go

    def sdpa_bwd(q, k, v, do, causal, gqa=False):
        leaves = [t.detach().requires_grad_(True) for t in (q, k, v)]
        with sdpa_kernel(fused_sdpa):
            out = F.scaled_dot_product_attention(*leaves, is_causal=causal, enable_gqa=gqa)

        def go():
            with sdpa_kernel(fused_sdpa):
                return torch.autograd.grad(out, leaves, do, retain_graph=True)
        return go

    def autograd_bwd(fn, inputs, grad_out, wrt):
        """Backward only: the graph of fn(*inputs) is built once and differentiated again."""
        leaves = [t.detach().requires_grad_(i in wrt) for i, t in enumerate(inputs)]
        out = fn(*leaves)
        targets = [leaves[i] for i in wrt]
        return lambda: torch.autograd.grad(out, targets, grad_out, retain_graph=True)

    def rotate_half(x, c, s_):
        x1, x2 = x.chunk(2, dim=-1)
        return torch.cat((x1 * c - x2 * s_, x2 * c + x1 * s_), dim=-1)

    g = torch.Generator(device=device).manual_seed(0)
    bf16 = torch.bfloat16
    # Config 1: softmax float32 [4096, 4096].
    x = torch.randn(4096, 4096, device=device, generator=g)

    def softmax_copy(i):
        xi = x if i == 0 else x.clone()
        yi = torch.empty_like(x)
        return lambda: sm._launch((xi,), yi)

    mem_row("tk_softmax_fwd", "f32 4096x4096", softmax_copy, 2 * x.numel() * 4, "1:1",
            ref="torch.softmax", size_matched=True,
            ref_make=lambda i: (lambda xi: lambda: torch.softmax(xi, -1))(x if i == 0 else x.clone()))
    del x
    # Online softmax (rows past the single-pass limit): f32 [64, 1048576], 64 chunks per row,
    # so the single-read kernel (one read, one write: the single-pass cost model).
    xw = torch.randn(64, 1 << 20, device=device, generator=g)

    def online_copy(i):
        xi = xw if i == 0 else xw.clone()
        yi = torch.empty_like(xw)
        return lambda: sm._launch_online((xi,), yi)

    mem_row("tk_softmax_online_fwd", "f32 64x1048576", online_copy, 2 * xw.numel() * 4, "1:1",
            ref="torch.softmax",
            ref_make=lambda i: (lambda xi: lambda: torch.softmax(xi, -1))(xw if i == 0 else xw.clone()))
    del xw
    # Config 3: SwiGLU bf16 [16384, 14336].
    gate = torch.randn(16384, 14336, device=device, dtype=bf16, generator=g)
    up = torch.randn(16384, 14336, device=device, dtype=bf16, generator=g)
    dy = torch.randn(16384, 14336, device=device, dtype=bf16, generator=g)
    out = torch.empty_like(gate)
    dv = torch.empty_like(gate)
    n = gate.numel()
    mem_row("tk_swiglu_fwd", "bf16 16384x14336",
            lambda i: (lambda: sg._launch_forward(up, gate, out)), 3 * n * 2, "2:1",
            ref="value * F.silu(gate)", ref_make=lambda i: (lambda: up * F.silu(gate)))
    mem_row("tk_swiglu_bwd", "bf16 16384x14336",
            lambda i: (lambda: sg._launch_backward_into(dy, up, gate, dv, out)), 5 * n * 2, "3:2",
            ref="autograd of value * F.silu(gate)",
            ref_make=lambda i: autograd_bwd(lambda v_, g_: v_ * F.silu(g_), (up, gate), dy, (0, 1)))
    del gate, up, dy, out, dv
    # Config 3: RoPE on q [4, 32, 4096, 128] viewed [524288, 128], per-row tables.
    q = torch.randn(4 * 32 * 4096, 128, device=device, dtype=bf16, generator=g)
    inv = 10000.0 ** (-torch.arange(0, 128, 2, device=device, dtype=torch.float32) / 128)
    ang = torch.arange(4096, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    cos = torch.cos(ang).to(bf16).repeat(128, 1)
    sin = torch.sin(ang).to(bf16).repeat(128, 1)

    def rope_copy(i, backward):
        qi, ci, si = (q, cos, sin) if i == 0 else (q.clone(), cos.clone(), sin.clone())
        out = torch.empty_like(q)
        if backward:
            return lambda: rp._launch_backward_into(qi, q, ci, si, out, None, None)
        return lambda: rp._launch_forward(qi, ci, si, out)

    mem_row("tk_rope_fwd", "bf16 [4,32,4096,128]", lambda i: rope_copy(i, False),
            3 * q.numel() * 2, "2:1", ref="rotate-half (torch.cat of x1*c - x2*s, x2*c + x1*s)",
            ref_make=lambda i: (lambda a: lambda: rotate_half(*a))(
                (q, cos, sin) if i == 0 else (q.clone(), cos.clone(), sin.clone())))
    mem_row("tk_rope_bwd", "bf16 [4,32,4096,128] dx only", lambda i: rope_copy(i, True),
            3 * q.numel() * 2, "2:1", ref="autograd of rotate-half, dx only",
            ref_make=lambda i: autograd_bwd(
                rotate_half, (q, cos, sin) if i == 0 else (q.clone(), cos.clone(), sin.clone()),
                q, (0,)))
    del q, cos, sin
    # GQA decode (reference decode model geometry Hq 32, Hkv 8, D 128; B 32, L 8192):
    # bytes = unique KV + Q + O (the model's Bytes_min).
    from tklab.kernels import gqa_decode as gd

    qd = torch.randn(32, 32, 128, device=device, dtype=bf16, generator=g)
    kd = torch.randn(32, 8, 8192, 128, device=device, dtype=bf16, generator=g)
    vd = torch.randn_like(kd)
    od = torch.empty_like(qd)
    lsed = torch.empty(32, 32, device=device)
    mem_row("tk_gqa_decode", "bf16 B32 Hq32 Hkv8 L8192 D128",
            lambda i: (lambda: gd._launch(qd, kd, vd, None, od, lsed, scale=128 ** -0.5)),
            2 * kd.numel() * 2 + 2 * qd.numel() * 2, "1:0", ref="SDPA (enable_gqa)",
            ref_make=lambda i: sdpa_fwd(qd[:, :, None], kd, vd, False, gqa=True))
    del qd, kd, vd, od, lsed
    # Config 4: GEMM.
    for dt_name, dt in (("float16", torch.float16), ("bfloat16", bf16)):
        for m, nn, k in ((8192, 8192, 8192), (4096, 4096, 4096), (8191, 8192, 8192)):
            if dt is bf16 and m != 8192:
                continue
            sc = k ** -0.25
            a = (torch.randn(m, k, device=device, generator=g) * sc).to(dt)
            b = (torch.randn(k, nn, device=device, generator=g) * sc).to(dt)
            c = torch.empty(m, nn, device=device, dtype=dt)
            mfma_row("tk_gemm", f"{dt_name} {m}x{nn}x{k}", lambda: mm._launch_fp32acc((a, b), c),
                     2 * m * nn * k, dt_name, ref="torch.mm (hipBLASLt)",
                     ref_fn=lambda: (lambda: torch.mm(a, b)))
            del a, b, c
    # Config 3 fused into its producer: the gate/up GEMM with SwiGLU in the epilogue,
    # x [16384, 4096] @ W_gate, W_up [4096, 14336] -> y [16384, 14336] (two GEMMs' FLOPs);
    # `unfused_ms` is two tk_gemm launches plus tk_swiglu_fwd on the same operands.
    from tklab.kernels import matmul_swiglu as mms
    from tklab.kernels import swiglu as sgl

    sc = 4096 ** -0.25
    xm = (torch.randn(16384, 4096, device=device, generator=g) * sc).to(bf16)
    wgm = (torch.randn(4096, 14336, device=device, generator=g) * sc).to(bf16)
    wum = (torch.randn(4096, 14336, device=device, generator=g) * sc).to(bf16)
    ym = torch.empty(16384, 14336, device=device, dtype=bf16)
    gm, um = torch.empty_like(ym), torch.empty_like(ym)
    timed_swiglu = mfma_row("tk_gemm_swiglu",
                            "bf16 16384x14336x4096 (gate+up GEMMs, SwiGLU epilogue)",
                            lambda: mms._launch(xm, wgm, wum, ym),
                            2 * 2 * 16384 * 14336 * 4096, "bfloat16", reps=5,
                            ref="torch.mm x2 + value * F.silu(gate)",
                            ref_fn=lambda: (lambda: torch.mm(xm, wum) * F.silu(torch.mm(xm, wgm))))

    def unfused():
        mm._launch_fp32acc((xm, wgm), gm)
        mm._launch_fp32acc((xm, wum), um)
        sgl._launch_forward(um, gm, ym)

    if timed_swiglu:
        rows[-1]["unfused_ms"] = round(timed(unfused, 5), 4)
    del xm, wgm, wum, ym, gm, um
    # Config 2 feeding its consumer: residual-RMSNorm then the grouped-query QKV
    # projection, x, r [16384, 4096] @ W [4096, 6144] (32 query + 2 x 8 KV heads of 128):
    # statistics pass + row-scaled GEMM on the folded weight (GEMM FLOPs);
    # `unfused_ms` is tk_rmsnorm_fwd writing s and y, then tk_gemm on y.
    from tklab.kernels import residual_rms_norm as rrn
    from tklab.kernels import rms_norm_matmul as rnm

    xq, rq = (torch.randn(16384, 4096, device=device, dtype=bf16, generator=g) for _ in range(2))
    wn = (1 + 0.02 * torch.randn(4096, device=device, generator=g)).to(bf16)
    wq = (torch.randn(4096, 6144, device=device, generator=g) * 4096 ** -0.5).to(bf16)
    wf = rnm.fold_norm_weight(wn, wq)
    timed_norm = mfma_row("residual_rms_norm_matmul (tk_rmsnorm_fwd stats + tk_gemm_rowscale)",
             "bf16 16384x6144x4096, residual add + RMSNorm in front",
             lambda: rnm.residual_rms_norm_matmul(xq, rq, wf, eps=1e-6),
             2 * 16384 * 6144 * 4096, "bfloat16", reps=5,
             ref="x + r, F.rms_norm, torch.mm",
             ref_fn=lambda: (lambda: torch.mm(F.rms_norm(xq + rq, (4096,), wn, 1e-6), wq)))
    sq, yq = torch.empty_like(xq), torch.empty_like(xq)
    rstdq = torch.empty(16384, device=device, dtype=torch.float32)
    cq = torch.empty(16384, 6144, device=device, dtype=bf16)

    def unfused_norm_gemm():
        rrn._launch_forward(xq, rq, wn, sq, yq, rstdq, eps=1e-6, store_residual=True,
                            store_stats=True)
        mm._launch_fp32acc((yq, wq), cq)

    if timed_norm:
        rows[-1]["unfused_ms"] = round(timed(unfused_norm_gemm, 5), 4)
        rows[-1]["fold_ms"] = round(timed(lambda: rnm.fold_norm_weight(wn, wq), 5), 4)
    del xq, rq, wq, wf, sq, yq, cq
    # Config 5: attention.
    for causal, nctx, d in ((True, 8192, 128), (False, 4096, 128), (True, 8192, 64), (False, 4096, 64)):
        shape = (4, 32, nctx, d)
        qq, kk, vv, do = (torch.randn(shape, device=device, dtype=bf16, generator=g) for _ in range(4))
        o = torch.empty_like(qq)
        lse = torch.empty(shape[:-1], device=device, dtype=torch.float32)
        delta = torch.empty_like(lse)
        gq, gk, gv = torch.empty_like(qq), torch.empty_like(qq), torch.empty_like(qq)
        flops = fa.attention_flops(4, 32, nctx, d, causal=causal)
        tag = f"bf16 B4 H32 N{nctx} D{d} {'causal' if causal else 'non-causal'}"
        mfma_row("tk_attn_fwd", tag,
                 lambda: fa._launch_forward(qq, kk, vv, o, lse, causal=causal, store_lse=True),
                 flops, "bfloat16", reps=5, ref="SDPA (flash/efficient backends)",
                 ref_fn=lambda: sdpa_fwd(qq, kk, vv, causal))
        mfma_row("tk_attn_bwd (preprocess+dkdv+dq)", tag + ", 2.5x fwd FLOPs",
                 lambda: fa._launch_backward_into(qq, kk, vv, o, lse, do, delta, gq, gk, gv,
                                                  causal=causal),
                 int(2.5 * flops), "bfloat16", reps=5, ref="SDPA backward (flash/efficient)",
                 ref_fn=lambda: sdpa_bwd(qq, kk, vv, do, causal))
        del qq, kk, vv, do, o, lse, delta, gq, gk, gv
    # Grouped-query attention at the causal config with 8 KV heads (4 query heads each).
    shape, kv_shape = (4, 32, 8192, 128), (4, 8, 8192, 128)
    qq, do = (torch.randn(shape, device=device, dtype=bf16, generator=g) for _ in range(2))
    kk, vv = (torch.randn(kv_shape, device=device, dtype=bf16, generator=g) for _ in range(2))
    o = torch.empty_like(qq)
    lse = torch.empty(shape[:-1], device=device, dtype=torch.float32)
    flops = fa.attention_flops(4, 32, 8192, 128, causal=True)
    tag = "bf16 B4 H32 Hkv8 N8192 D128 causal"
    mfma_row("tk_attn_fwd_gqa", tag,
             lambda: fa._launch_gqa_forward(qq, kk, vv, o, lse, causal=True), flops, "bfloat16",
             reps=5, ref="SDPA (enable_gqa)", ref_fn=lambda: sdpa_fwd(qq, kk, vv, True, gqa=True))
    mfma_row("tk_attn_bwd_gqa (preprocess+dkdv+dq)", tag + ", 2.5x fwd FLOPs",
             lambda: fa._launch_gqa_backward(qq, kk, vv, o, lse, do, causal=True),
             int(2.5 * flops), "bfloat16", reps=5, ref="SDPA backward (enable_gqa)",
             ref_fn=lambda: sdpa_bwd(qq, kk, vv, do, True, gqa=True))
    # RoPE in the attention prologue: position tables [8192, 64] (base 1e4); Q rotated
    # as the forward loads it, K rotated once into a workspace. `unfused_ms` is the RoPE
    # kernel on Q and on K, then the plain forward on the rotated tensors.
    inv_f = 10000.0 ** (-torch.arange(64, dtype=torch.float32) / 64)
    ang = torch.arange(8192, dtype=torch.float32)[:, None] * inv_f[None]
    rcos, rsin = ang.cos().to(bf16).to(device), ang.sin().to(bf16).to(device)
    kr, qr = torch.empty_like(kk), torch.empty_like(qq)
    timed_rope = mfma_row("tk_attn_fwd_rope", tag + ", RoPE on Q (prologue) and K",
             lambda: fa._launch_rope_forward(qq, kk, vv, rcos, rsin, o, lse, kr, causal=True),
             flops, "bfloat16", reps=5)

    def unfused_rope():
        fa._rope_positions(qq, rcos, rsin, qr, inverse=False)
        fa._rope_positions(kk, rcos, rsin, kr, inverse=False)
        fa._launch_gqa_forward(qr, kr, vv, o, lse, causal=True)

    if timed_rope:
        rows[-1]["unfused_ms"] = round(timed(unfused_rope, 5), 4)
    del qq, kk, vv, do, o, lse, kr, qr
    # Variable-length causal attention: one packed batch of 32768 tokens in sequences of
    # 8192, 2 x 4096, 4 x 2048 and 8 x 1024 (H32 Hkv8 D128); FLOPs summed per sequence.
    lengths = [8192] + [4096] * 2 + [2048] * 4 + [1024] * 8
    total = sum(lengths)
    cu = torch.tensor([0] + list(itertools.accumulate(lengths)), device=device,
                      dtype=torch.int32)
    qq, do = (torch.randn(total, 32, 128, device=device, dtype=bf16, generator=g)
              for _ in range(2))
    kk, vv = (torch.randn(total, 8, 128, device=device, dtype=bf16, generator=g)
              for _ in range(2))
    o = torch.empty_like(qq)
    lse = torch.empty(32, total, device=device, dtype=torch.float32)
    flops = sum(fa.attention_flops(1, 32, n, 128, causal=True) for n in lengths)
    tag = "bf16 H32 Hkv8 D128 causal, 32768 tokens in 15 sequences of 1024-8192"
    mfma_row("tk_attn_fwd_varlen", tag,
             lambda: fa._launch_varlen_forward(qq, kk, vv, cu, 8192, o, lse, causal=True),
             flops, "bfloat16", reps=5)
    mfma_row("tk_attn_bwd_varlen (preprocess+dkdv+dq)", tag + ", 2.5x fwd FLOPs",
             lambda: fa._launch_varlen_backward(qq, kk, vv, cu, 8192, o, lse, do, causal=True),
             int(2.5 * flops), "bfloat16", reps=5)
    del qq, kk, vv, do, o, lse, cu
    del flush
    torch.cuda.empty_cache()
    return rows


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build's kernels shard rows/heads with no "
              "exchange, and no multi-GPU figure is produced (run with --gpus 1).", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    step = Step(torch, device)
    ms_step, dominant, dominant_ms, attribution = time_step(torch, step, args.steps, args.warmup)
    step_bytes = sum(STEP_BYTES.values())
    value = step_bytes / (ms_step / 1e3) / 1e9
    progress(f"step {ms_step:.4f} ms ({value:.1f} GB/s), {dominant} {dominant_ms:.5f} ms")
    ref_step_ms = torch_gpu_step_ms(torch, step, max(10, args.steps // 4))

    achieved = STEP_BYTES[dominant] / (dominant_ms / 1e3) / 1e9
    traffic = _traffic_from_summary() if dominant == "tk_rmsnorm_bwd_stage1" else None
    roofline = {
        "bound": "hbm",
        "kernel": dominant,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBPS, 4),
        "traffic": traffic,
        "algorithmic_bytes": STEP_BYTES[dominant],
        "kernel_ms": round(dominant_ms, 5),
        "attribution_ms": {k: round(v, 5) for k, v in attribution.items()},
    }
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch.randn on device)",
        "config": {
            "workload": "residual_rms_norm forward+backward (benchmark config 2)",
            "rows": ROWS,
            "cols": COLS,
            "eps": EPS,
            "bytes_per_step": step_bytes,
        },
        "roofline": roofline,
        "reference_gpu": {
            "impl": "torch (x + r, F.rms_norm, torch.autograd.grad), bf16 on this GPU",
            "ms_per_step": round(ref_step_ms, 5),
            "value": round(step_bytes / (ref_step_ms / 1e3) / 1e9, 1),
            "speedup": round(ref_step_ms / ms_step, 3),
        },
    }
    del step
    torch.cuda.empty_cache()
    roofs = measured_roofs(torch, device)
    progress(f"measured roofs: HBM {roofs['hbm_GBps']} GB/s")
    line["measured_roofs"] = roofs
    roofline["measured_peak"] = roofs["hbm_GBps"]
    roofline["frac_measured"] = round(achieved / roofs["hbm_GBps"], 4)
    # Stage 1 reads dy, s and the incoming sum gradient and writes dx: a 3:1 stream.
    mix = {"tk_rmsnorm_bwd_stage1": "3:1", "tk_rmsnorm_fwd": "2:2"}.get(dominant)
    if mix:
        roofline["mix"] = mix
        roofline["frac_mix"] = round(achieved / roofs["stream_mixes_GBps"][mix], 4)
    if not args.no_kernels:
        line["kernels"] = kernel_table(torch, device, roofs, args.only)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch)
        progress(f"cpu baseline {line['cpu_baseline']['value']} GB/s")
        line["cpu_oracle_port"] = cpu_oracle_port(args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
