"""Registry-wide GPU correctness: every spec, dtype and validation size.

Same procedure as the reference's tests/test_correctness.py: seed 0, build the
spec's inputs, run the entry point, compare with the spec's PyTorch reference
evaluated on float32 upcasts (the spec's assert_fn, else the dtype tolerance
table), for the allocation-free launcher and the naive baseline too, then the
adversarial case.
"""

from __future__ import annotations

import pytest
import torch

import tklab.kernels  # noqa: F401
from tklab.harness.tolerances import assert_close
from tklab.registry import REGISTRY, KernelSpec

pytestmark = pytest.mark.gpu


def _check(spec: KernelSpec, output: torch.Tensor, reference: torch.Tensor) -> None:
    if spec.assert_fn is None:
        assert_close(output, reference, rtol=spec.rtol, atol=spec.atol)
    else:
        spec.assert_fn(output, reference)


@pytest.mark.parametrize("name", sorted(REGISTRY))
def test_spec_matches_its_reference(name: str) -> None:
    spec = REGISTRY[name]
    device = torch.device("cuda")
    torch.manual_seed(0)
    for dtype in spec.dtypes:
        for size in spec.validation_sizes():
            args = spec.make_inputs(size, device, dtype)
            reference = spec.ref_fn(*(a.float() for a in args))
            _check(spec, spec.triton_fn(*args), reference)
            # The naive baselines are unfused PyTorch compositions in the storage
            # dtype; in bfloat16 their intermediate roundings (e.g. two products
            # that cancel in RoPE) exceed the table, so they are checked in the
            # dtypes the reference registered them for (float16/float32).
            if spec.naive_fn is not None and dtype != torch.bfloat16:
                _check(spec, spec.naive_fn(*args), reference)
            out = spec.make_output(args)
            spec.launch_fn(args, out)
            _check(spec, out, reference)
    if spec.make_adversarial is not None:
        args = spec.make_adversarial(device)
        reference = spec.ref_fn(*(a.float() for a in args))
        _check(spec, spec.triton_fn(*args), reference)
