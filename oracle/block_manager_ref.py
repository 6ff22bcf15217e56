"""Plain-Python restatement of the reference BlockManager (test infrastructure only).

Follows nv/npu/block_manager.py:1-328 step by step, with Python lists for the
free queue (pop from the front, append on release, remove on retain) and
nested (parent, token tuple) keys for the prefix cache, exactly as the
reference does, and builds metadata with the per-token slot loop the GPU
packing replaces.  Metadata tensors are returned on the CPU.

Pins (tests/test_oracle.py): the reference's three known-answer tests
(tests/test_block_manager.py:6-54) and golden traces written from the
reference source by tests/golden/make_block_traces.py.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class MetadataRef:
    """PagedKVCacheMetadata (nv/npu/block_manager.py:12-20), all on the CPU."""

    block_tables: torch.Tensor
    context_lens: torch.Tensor
    slot_mapping: torch.Tensor
    actual_seq_lengths_q: list[int] | None = None
    actual_seq_lengths_kv: list[int] | None = None
    query_lens: list[int] | None = None
    use_paged_prefill: bool = False


@dataclass
class _Block:
    block_id: int
    ref_count: int = 0
    block_hash: object = None


class BlockManagerRef:
    def __init__(self, num_blocks: int, block_size: int):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.blocks = [_Block(i) for i in range(num_blocks)]
        self.free_block_ids: list[int] = list(range(num_blocks))  # nv/npu/block_manager.py:49
        self.cached_block_hash_to_ids: dict = {}
        self.block_tables: dict[int, list[int]] = {}
        self.seq_lens: dict[int, int] = {}

    # -- hashing (nv/npu/block_manager.py:54-65) --
    def _key(self, token_ids, block_idx, parent):
        lo = block_idx * self.block_size
        toks = token_ids[lo : lo + self.block_size]
        toks = toks.tolist() if hasattr(toks, "tolist") else list(toks)
        return (parent, tuple(int(t) for t in toks))

    # -- pool (nv/npu/block_manager.py:67-112) --
    def _evict(self, block_id):
        blk = self.blocks[block_id]
        if blk.block_hash is None:
            return
        ids = self.cached_block_hash_to_ids[blk.block_hash]
        ids.remove(block_id)
        if not ids:
            del self.cached_block_hash_to_ids[blk.block_hash]
        blk.block_hash = None

    def _alloc_block(self) -> int:
        if not self.free_block_ids:
            raise RuntimeError("BlockManager out of free blocks")
        block_id = self.free_block_ids.pop(0)
        self._evict(block_id)
        blk = self.blocks[block_id]
        if blk.ref_count != 0:
            raise RuntimeError(f"block {block_id} is not free")
        blk.ref_count = 1
        return block_id

    def _retain_block(self, block_id):
        blk = self.blocks[block_id]
        if blk.ref_count == 0:
            self.free_block_ids.remove(block_id)
        blk.ref_count += 1

    def _release_block(self, block_id):
        blk = self.blocks[block_id]
        if blk.ref_count <= 0:
            raise RuntimeError(f"block {block_id} ref_count underflow")
        blk.ref_count -= 1
        if blk.ref_count == 0:
            self.free_block_ids.append(block_id)

    def _required(self, end_pos):
        return 0 if end_pos <= 0 else math.ceil(end_pos / self.block_size)

    # -- sequences (nv/npu/block_manager.py:114-185) --
    def _init_slot(self, slot, start_pos, prefix_block_ids):
        if slot in self.block_tables:
            return
        table = list(prefix_block_ids or [])
        for b in table:
            self._retain_block(b)
        self.block_tables[slot] = table
        self.seq_lens[slot] = start_pos

    def ensure_blocks(self, slot, end_pos):
        table = self.block_tables[slot]
        while len(table) < self._required(end_pos):
            table.append(self._alloc_block())

    def find_longest_prefix_blocks(self, token_ids, max_cache_blocks):
        found, parent = [], None
        for i in range(max_cache_blocks):
            key = self._key(token_ids, i, parent)
            ids = self.cached_block_hash_to_ids.get(key)
            if not ids:
                break
            found.append(ids[0])
            parent = key
        return found

    def cache_full_blocks(self, slot, token_ids, num_cached_blocks=0, num_full_blocks=None):
        table = self.block_tables[slot]
        n_full = num_full_blocks
        if n_full is None:
            n_full = int(token_ids.numel() if hasattr(token_ids, "numel") else len(token_ids)) // self.block_size
        parent = self.blocks[table[num_cached_blocks - 1]].block_hash if num_cached_blocks > 0 else None
        for i in range(num_cached_blocks, n_full):
            blk = self.blocks[table[i]]
            if blk.block_hash is not None:
                parent = blk.block_hash
                continue
            key = self._key(token_ids, i, parent)
            blk.block_hash = key
            self.cached_block_hash_to_ids.setdefault(key, []).append(blk.block_id)
            parent = key

    def free_slot(self, slot):
        table = self.block_tables.pop(slot, [])
        self.seq_lens.pop(slot, None)
        for b in reversed(table):
            self._release_block(b)

    def clear_prefix_cache(self):
        if self.block_tables or any(b.ref_count > 0 for b in self.blocks):
            raise RuntimeError("cannot clear prefix cache with active sequences")
        self.cached_block_hash_to_ids.clear()
        for b in self.blocks:
            b.block_hash = None

    # -- metadata (nv/npu/block_manager.py:194-328) --
    def _physical_slot(self, slot, pos):
        table = self.block_tables[slot]
        idx = pos // self.block_size
        if idx >= len(table):
            raise RuntimeError(f"missing block: slot={slot}, logical_pos={pos}")
        return table[idx] * self.block_size + pos % self.block_size

    def get_block_tables_tensor(self, slots):
        width = max(len(self.block_tables[s]) for s in slots)
        out = torch.zeros((len(slots), width), dtype=torch.int32)
        for i, s in enumerate(slots):
            t = self.block_tables[s]
            out[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
        return out

    def get_context_lens_tensor(self, slots):
        return torch.tensor([self.seq_lens[s] for s in slots], dtype=torch.int32)

    def get_slot_mapping(self, slots, start_positions, num_tokens_per_seq):
        mapping = []
        for s, start, n in zip(slots, start_positions, num_tokens_per_seq):
            for k in range(n):
                mapping.append(self._physical_slot(s, start + k))
        return torch.tensor(mapping, dtype=torch.int64)

    def prepare_prefill_metadata(self, slots, seq_lens, start_positions, prefix_block_ids):
        if not (len(slots) == len(seq_lens) == len(start_positions) == len(prefix_block_ids)):
            raise ValueError("slots, seq_lens, start_positions and prefix_block_ids length mismatch")
        q_cum, kv_cum, tq, tkv = [], [], 0, 0
        for s, n, start, prefix in zip(slots, seq_lens, start_positions, prefix_block_ids):
            self._init_slot(s, start, prefix)
            end = start + n
            self.ensure_blocks(s, end)
            self.seq_lens[s] = max(self.seq_lens[s], end)
            tq += n
            tkv += end
            q_cum.append(tq)
            kv_cum.append(tkv)
        return MetadataRef(
            block_tables=self.get_block_tables_tensor(slots),
            context_lens=self.get_context_lens_tensor(slots),
            slot_mapping=self.get_slot_mapping(slots, start_positions, seq_lens),
            actual_seq_lengths_q=q_cum,
            actual_seq_lengths_kv=kv_cum,
            query_lens=list(seq_lens),
            use_paged_prefill=any(p > 0 for p in start_positions),
        )

    def prepare_decode_metadata(self, slots, start_positions, q_len):
        if len(slots) != len(start_positions):
            raise ValueError("slots and start_positions length mismatch")
        for s, start in zip(slots, start_positions):
            end = start + q_len
            self.ensure_blocks(s, end)
            self.seq_lens[s] = max(self.seq_lens[s], end)
        return MetadataRef(
            block_tables=self.get_block_tables_tensor(slots),
            context_lens=self.get_context_lens_tensor(slots),
            slot_mapping=self.get_slot_mapping(slots, start_positions, [q_len] * len(slots)),
        )


__all__ = ["BlockManagerRef", "MetadataRef"]
