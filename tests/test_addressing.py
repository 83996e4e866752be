"""int32 offset guard (known answers of the reference's tests/test_addressing.py)."""

from __future__ import annotations

import pytest
import torch

from tklab.harness.addressing import MAX_INT32_OFFSET, assert_int32_addressable, max_relative_offset


def test_extent_of_dense_and_broadcast_layouts() -> None:
    assert max_relative_offset(torch.empty_strided((3, 5), (5, 1), device="meta")) == 14
    assert max_relative_offset(torch.empty_strided((3, 5), (0, 1), device="meta")) == 4


def test_empty_tensor_has_no_extent() -> None:
    assert max_relative_offset(torch.empty_strided((0, 2), (2**31, 1), device="meta")) == 0


def test_negative_strides_count_by_magnitude() -> None:
    assert max_relative_offset(torch.empty(4, 3).flip(0)) == 3 * 3 + 2


def test_boundary_is_inclusive() -> None:
    ok = torch.empty_strided((2, 1), (MAX_INT32_OFFSET, 1), device="meta")
    assert_int32_addressable(ok, name="edge")
    too_far = torch.empty_strided((2, 2), (2**31, 1), device="meta")
    with pytest.raises(ValueError, match="int32 offset"):
        assert_int32_addressable(too_far, name="test tensor")
