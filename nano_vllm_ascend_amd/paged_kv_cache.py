"""Paged KV store (nv/npu/paged_kv_cache.py:1-72).

Two bf16 tensors [num_layers, num_blocks, block_size, num_kv_heads, head_dim],
allocated once; ``write`` scatters token rows into slots with the HIP store
kernel (the reference used two index_copy_ calls) and ``get_physical_cache``
hands out per-layer [num_blocks, block_size, num_kv_heads, head_dim] views.
At 128-token pages one block of K for one layer is 128 * 8 * 128 * 2 B =
256 KiB of contiguous HBM, so a page is read with long linear bursts.
"""
from __future__ import annotations

import torch

from . import _C


class PagedKVCache:
    def __init__(self, num_layers: int, num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                 dtype: torch.dtype, device):
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        self.key_cache = torch.empty(shape, dtype=dtype, device=device)
        self.value_cache = torch.empty(shape, dtype=dtype, device=device)

    @staticmethod
    def bytes_per_block(num_layers: int, block_size: int, num_kv_heads: int, head_dim: int, elem: int = 2) -> int:
        return 2 * num_layers * block_size * num_kv_heads * head_dim * elem

    def write(self, layer_idx: int, key_states: torch.Tensor, value_states: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
        total, hkv, d = key_states.shape
        if hkv != self.num_kv_heads or d != self.head_dim:
            raise ValueError(f"kv shape mismatch: got {tuple(key_states.shape)}")
        if slot_mapping.numel() != total:
            raise ValueError(f"slot_mapping numel {slot_mapping.numel()} != total_tokens {total}")
        slots = slot_mapping.to(device=self.key_cache.device, dtype=torch.int64)
        _C.kv_cache_write(key_states, value_states, self.key_cache[layer_idx], self.value_cache[layer_idx], slots)

    def get_physical_cache(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        return self.key_cache[layer_idx], self.value_cache[layer_idx]
