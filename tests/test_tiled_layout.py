"""The tiled operand layout of the skinny GEMM (include/nvamd.h, "Tiled layout"), on the CPU.

_C.tile / _C.untile are plain torch reshapes; the kernels address the same layout with
tiled_index().  Element (r, c) of a [R, C] matrix must sit at
((r/16) * (C/32) + c/32) * 512 + 128 * ((c%32)/8) + 8 * (r%16) + c%8, the formula written out
here independently of both.
"""
from __future__ import annotations

import pytest
import torch

from nano_vllm_ascend_amd import _C


def _index(r, c, cols):
    return ((r // 16) * (cols // 32) + c // 32) * 512 + 128 * ((c % 32) // 8) + 8 * (r % 16) + c % 8


@pytest.mark.parametrize("rows,cols", [(1, 32), (16, 64), (17, 96), (32, 1024), (40, 128)])
def test_tile_places_every_element_at_the_documented_index(rows, cols):
    a = torch.arange(rows * cols, dtype=torch.int32).reshape(rows, cols)  # exact values
    t = _C.tile(a)
    assert t.shape == (-(-rows // 16), cols // 32, 512) and t.is_contiguous()
    flat = t.reshape(-1)
    r = torch.arange(rows).view(-1, 1).expand(rows, cols)
    c = torch.arange(cols).view(1, -1).expand(rows, cols)
    idx = _index(r, c, cols)
    assert torch.equal(flat[idx.reshape(-1)], a.reshape(-1))
    # padding rows (up to a multiple of 16) are zero
    pad = 16 * t.shape[0] - rows
    assert pad == 0 or int(_C.untile(t)[rows:].abs().sum()) == 0


def test_untile_inverts_tile():
    gen = torch.Generator().manual_seed(0)
    a = torch.randn(27, 256, generator=gen).to(torch.bfloat16)
    assert torch.equal(_C.untile(_C.tile(a), 27), a)
    assert _C.untile(_C.tile(a)).shape == (32, 256)


def test_lane_holds_eight_consecutive_columns():
    """MFMA lane l = n + 16 g of a tile reads its 8 elements at 8 l: row n, columns 8g..8g+7."""
    a = torch.arange(16 * 32, dtype=torch.int32).reshape(16, 32)
    t = _C.tile(a).reshape(512)
    for lane in range(64):
        n, g = lane % 16, lane // 16
        assert torch.equal(t[8 * lane : 8 * lane + 8], a[n, 8 * g : 8 * g + 8])


def test_tile_rejects_columns_not_a_multiple_of_32():
    with pytest.raises(ValueError):
        _C.tile(torch.zeros(4, 40))
    with pytest.raises(ValueError):
        _C.untile(torch.zeros(4, 40))
