"""Host-side range checks (CPU): indices the reference's torch indexing would reject raise IndexError.

The kernels clamp or skip such indices; with range checks on, the eager wrappers call these
functions first.  They are plain tensor code, so they are tested here on CPU tensors; the GPU
test in test_paged_decode_gpu.py checks a wrapper raising through them.
"""
from __future__ import annotations

import pytest
import torch

from nano_vllm_ascend_amd import _C


def test_positions_inside_the_rope_table():
    _C.check_positions(torch.tensor([0, 5, 4095]), 4096)
    with pytest.raises(IndexError):
        _C.check_positions(torch.tensor([0, 4096]), 4096)
    with pytest.raises(IndexError):
        _C.check_positions(torch.tensor([-1]), 4096)
    _C.check_positions(torch.tensor([], dtype=torch.int64), 4096)


def test_slots_inside_the_cache_or_padding():
    _C.check_slots(torch.tensor([0, 7, -1, 1023]), 1024)  # -1: a padding row, not stored
    with pytest.raises(IndexError):
        _C.check_slots(torch.tensor([1024]), 1024)
    with pytest.raises(IndexError):
        _C.check_slots(torch.tensor([3, -2]), 1024)


def test_contexts_fit_their_table_row_and_pool():
    bt = torch.tensor([[3, 1, 0], [2, 0, 0]], dtype=torch.int32)
    _C.check_paged_context(bt, torch.tensor([300, 100], dtype=torch.int32), num_blocks=4, block_size=128,
                           max_context_len=384)
    with pytest.raises(IndexError):  # longer than the table row
        _C.check_paged_context(bt, torch.tensor([385, 1], dtype=torch.int32), 4, 128)
    with pytest.raises(IndexError):  # longer than the launch bound
        _C.check_paged_context(bt, torch.tensor([300, 1], dtype=torch.int32), 4, 128, max_context_len=256)
    with pytest.raises(IndexError):  # a used entry names a block outside the pool
        _C.check_paged_context(torch.tensor([[9, 0]], dtype=torch.int32), torch.tensor([5], dtype=torch.int32), 4,
                               128)
    _C.check_paged_context(torch.tensor([[9, 0]], dtype=torch.int32), torch.tensor([0], dtype=torch.int32), 4, 128)


def test_checks_are_off_by_default_and_switchable(monkeypatch):
    monkeypatch.setattr(_C, "_range_checks", False)
    assert not _C._checking()
    prev = _C.set_range_checks(True)
    try:
        assert prev is False and _C._checking()
    finally:
        _C.set_range_checks(prev)
