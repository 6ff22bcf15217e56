"""Block pool, prefix cache and GPU-packed paged-KV metadata (nv/npu/block_manager.py:1-328).

The allocation state machine is the reference's, decision for decision:
  - the free queue pops from the front, appends on release and drops a block
    when a prefix hit retains it (an insertion-ordered dict gives the same
    order as the reference's list with O(1) operations);
  - ``free_slot`` releases a table in reverse;
  - a prefix-cache key is the chain (parent key, 128 token ids); a cached
    block keeps its key while it sits free and loses it only when it is
    re-allocated (lazy eviction).  Keys are interned to integers: two chains
    get the same integer exactly when the reference's nested tuples compare
    equal, so lookups hit and miss identically.

What moves to the GPU is building the metadata tensors.  Each live sequence
owns a row of a device-resident block-table mirror; table entries that change
are queued and shipped with the per-sequence descriptors in a single
host-to-device transfer, and ``nvamd_pack_batch`` expands them into
block_tables, context_lens, slot_mapping, positions, cu_seqlens,
last_token_indices and input_ids.  The reference instead ran a per-token
Python loop for slot_mapping and one host-to-device copy per table row.
"""
from __future__ import annotations

import math
from collections import OrderedDict
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _C


@dataclass
class PagedKVCacheMetadata:
    """The packed-batch contract handed to attention (nv/npu/block_manager.py:12-20).

    Differences from the reference: ``context_lens`` is on the DEVICE (the
    decode kernel reads it there, so a captured graph needs no host update);
    its host copy is ``context_lens_host``.  The remaining fields after
    ``use_paged_prefill`` are produced by the same packing kernel.
    """

    block_tables: torch.Tensor
    context_lens: torch.Tensor
    slot_mapping: torch.Tensor
    actual_seq_lengths_q: list[int] | None = None
    actual_seq_lengths_kv: list[int] | None = None
    query_lens: list[int] | None = None
    use_paged_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None        # int32 [B+1]
    positions: torch.Tensor | None = None           # int64 [T]
    last_token_indices: torch.Tensor | None = None  # int64 [B]
    input_ids: torch.Tensor | None = None           # int64 [T]
    context_lens_host: list[int] = field(default_factory=list)
    max_context_len: int = 0
    max_query_len: int = 0
    # decode: grid bound of the paged kernel (a captured graph fixes it) and its workspace
    max_context_bound: int | None = None
    decode_workspace: torch.Tensor | None = None


@dataclass
class BlockState:
    block_id: int
    ref_count: int = 0
    block_hash: int | None = None


class _Uploader:
    """Two pinned host buffers used alternately, feeding one device int32 buffer."""

    def __init__(self, device, capacity: int = 1 << 14):
        self.device = device
        self._alloc(capacity)

    def _alloc(self, capacity: int) -> None:
        self.capacity = capacity
        self.host = [torch.empty(capacity, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self.host_np = [h.numpy() for h in self.host]
        self.dev = torch.empty(capacity, dtype=torch.int32, device=self.device)
        self.events: list[torch.cuda.Event | None] = [None, None]
        self.k = 0

    def upload(self, arr: np.ndarray) -> torch.Tensor:
        n = int(arr.size)
        if n > self.capacity:
            torch.cuda.current_stream().synchronize()
            self._alloc(max(n, 2 * self.capacity))
        k = self.k
        self.k ^= 1
        if self.events[k] is not None:
            self.events[k].synchronize()  # the copy that last read this host buffer is done
        self.host_np[k][:n] = arr
        self.dev[:n].copy_(self.host[k][:n], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self.events[k] = ev
        return self.dev


class BlockManager:
    """Unified block pool for runtime allocation and prefix-cache reuse.

    Prefix-cached blocks stay in the free queue when their ref_count reaches
    zero; their key is dropped only when the block is re-allocated.
    """

    def __init__(self, num_blocks: int, block_size: int, device, max_seqs: int = 64,
                 max_blocks_per_seq: int = 64):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.device = torch.device(device)
        self.blocks = [BlockState(i) for i in range(num_blocks)]
        self._free: OrderedDict[int, None] = OrderedDict.fromkeys(range(num_blocks))
        self.cached_block_hash_to_ids: dict[int, list[int]] = {}
        self._key_ids: dict[tuple, int] = {}
        self.block_tables: dict[int, list[int]] = {}
        self.seq_lens: dict[int, int] = {}
        # device mirror
        self._row_of: dict[int, int] = {}
        self._free_rows: list[int] = []
        self._rows_used = 0
        self._pending: dict[tuple[int, int], int] = {}
        self._mirror: torch.Tensor | None = None
        self._mirror_rows = max(1, max_seqs)
        self._mirror_width = max(1, max_blocks_per_seq)
        self._uploader: _Uploader | None = None

    # ------------------------------------------------------------------ pool
    @property
    def free_block_ids(self) -> list[int]:
        return list(self._free)

    def _token_tuple(self, token_ids, start: int, end: int) -> tuple[int, ...]:
        part = token_ids[start:end]
        if hasattr(part, "tolist"):
            part = part.tolist()
        return tuple(int(t) for t in part)

    def _key_id(self, parent: int | None, tokens: tuple[int, ...], create: bool) -> int | None:
        key = (parent, tokens)
        kid = self._key_ids.get(key)
        if kid is None and create:
            kid = len(self._key_ids)
            self._key_ids[key] = kid
        return kid

    def _evict_block_hash(self, block_id: int) -> None:
        block = self.blocks[block_id]
        if block.block_hash is None:
            return
        ids = self.cached_block_hash_to_ids[block.block_hash]
        ids.remove(block_id)
        if not ids:
            del self.cached_block_hash_to_ids[block.block_hash]
        block.block_hash = None

    def _alloc_block(self) -> int:
        if not self._free:
            raise RuntimeError("BlockManager out of free blocks")
        block_id, _ = self._free.popitem(last=False)
        self._evict_block_hash(block_id)
        block = self.blocks[block_id]
        if block.ref_count != 0:
            raise RuntimeError(f"block {block_id} is not free")
        block.ref_count = 1
        return block_id

    def _retain_block(self, block_id: int) -> None:
        block = self.blocks[block_id]
        if block.ref_count == 0:
            del self._free[block_id]
        block.ref_count += 1

    def _release_block(self, block_id: int) -> None:
        block = self.blocks[block_id]
        if block.ref_count <= 0:
            raise RuntimeError(f"block {block_id} ref_count underflow")
        block.ref_count -= 1
        if block.ref_count == 0:
            self._free[block_id] = None

    def _num_required_blocks(self, end_pos: int) -> int:
        return math.ceil(end_pos / self.block_size) if end_pos > 0 else 0

    # ------------------------------------------------------------- sequences
    def _assign_row(self, slot: int) -> int:
        if self._free_rows:
            row = self._free_rows.pop()
        else:
            row = self._rows_used
            self._rows_used += 1
        self._row_of[slot] = row
        return row

    def _init_slot(self, slot: int, start_pos: int, prefix_block_ids: list[int]) -> None:
        if slot in self.block_tables:
            return
        table = list(prefix_block_ids or [])
        for block_id in table:
            self._retain_block(block_id)
        self.block_tables[slot] = table
        self.seq_lens[slot] = start_pos
        row = self._assign_row(slot)
        for col, block_id in enumerate(table):
            self._pending[(row, col)] = block_id

    def ensure_blocks(self, slot: int, end_pos: int) -> None:
        table = self.block_tables[slot]
        need = self._num_required_blocks(end_pos)
        if len(table) >= need:
            return
        row = self._row_of[slot]
        while len(table) < need:
            block_id = self._alloc_block()
            self._pending[(row, len(table))] = block_id
            table.append(block_id)

    def find_longest_prefix_blocks(self, token_ids, max_cache_blocks: int) -> list[int]:
        found: list[int] = []
        parent: int | None = None
        bs = self.block_size
        for i in range(max_cache_blocks):
            kid = self._key_id(parent, self._token_tuple(token_ids, i * bs, (i + 1) * bs), create=False)
            ids = self.cached_block_hash_to_ids.get(kid) if kid is not None else None
            if not ids:
                break
            found.append(ids[0])
            parent = kid
        return found

    def cache_full_blocks(self, slot: int, token_ids, num_cached_blocks: int = 0,
                          num_full_blocks: int | None = None) -> None:
        table = self.block_tables[slot]
        n_full = num_full_blocks
        if n_full is None:
            n_full = (int(token_ids.numel()) if hasattr(token_ids, "numel") else len(token_ids)) // self.block_size
        parent = self.blocks[table[num_cached_blocks - 1]].block_hash if num_cached_blocks > 0 else None
        bs = self.block_size
        for i in range(num_cached_blocks, n_full):
            block = self.blocks[table[i]]
            if block.block_hash is not None:
                parent = block.block_hash
                continue
            kid = self._key_id(parent, self._token_tuple(token_ids, i * bs, (i + 1) * bs), create=True)
            block.block_hash = kid
            self.cached_block_hash_to_ids.setdefault(kid, []).append(block.block_id)
            parent = kid

    def free_slot(self, slot: int) -> None:
        table = self.block_tables.pop(slot, [])
        self.seq_lens.pop(slot, None)
        for block_id in reversed(table):
            self._release_block(block_id)
        row = self._row_of.pop(slot, None)
        if row is not None:
            self._free_rows.append(row)

    def clear_prefix_cache(self) -> None:
        if self.block_tables or any(block.ref_count > 0 for block in self.blocks):
            raise RuntimeError("cannot clear prefix cache with active sequences")
        self.cached_block_hash_to_ids.clear()
        self._key_ids.clear()
        for block in self.blocks:
            block.block_hash = None

    def _physical_slot(self, slot: int, logical_pos: int) -> int:
        table = self.block_tables[slot]
        idx = logical_pos // self.block_size
        if idx >= len(table):
            raise RuntimeError(f"missing block: slot={slot}, logical_pos={logical_pos}")
        return table[idx] * self.block_size + logical_pos % self.block_size

    # --------------------------------------------------------- GPU packing
    def _ensure_mirror(self, extra_width: int = 0) -> torch.Tensor:
        """Device mirror [rows, width]; doubles a dimension (keeping its contents) when outgrown."""
        need_rows = max(self._rows_used, 1)
        need_width = max([len(t) for t in self.block_tables.values()] + [1]) + extra_width
        m = self._mirror
        if m is not None and m.shape[0] >= need_rows and m.shape[1] >= need_width:
            return m
        rows, width = (self._mirror_rows, self._mirror_width) if m is None else tuple(m.shape)
        while rows < need_rows:
            rows *= 2
        while width < need_width:
            width *= 2
        new = torch.zeros((rows, width), dtype=torch.int32, device=self.device)
        if m is not None:
            new[: m.shape[0], : m.shape[1]].copy_(m)
        self._mirror = new
        return new

    def _pack(self, slots, starts, qlens, token_ids=None, width: int | None = None,
              out=None, tentative: dict[tuple[int, int], int] | None = None) -> PagedKVCacheMetadata:
        """Ship descriptors + pending table entries (+ token ids) and expand them on the GPU.

        ``tentative`` maps (row, column) to blocks a decode step packed ahead of time will use
        but the pool has not handed out yet: they are shipped and counted in the step's tables
        and context lengths, and the host state is left as it is.
        """
        b = len(slots)
        bs = self.block_size
        nblk = [len(self.block_tables[s]) for s in slots]
        # a step's context ends at its last token; the recorded length already covers it, except
        # for a step packed ahead of its confirmation
        ctx = [max(self.seq_lens[s], st + n) for s, st, n in zip(slots, starts, qlens)]
        if tentative:
            extra_cols = {row: col for row, col in tentative}
            for i, s in enumerate(slots):
                col = extra_cols.get(self._row_of[s])
                if col is not None:
                    nblk[i] = col + 1
        for s, start, n, nb in zip(slots, starts, qlens, nblk):
            if start + n > nb * bs:
                raise RuntimeError(f"missing block: slot={s}, logical_pos={start + n - 1}")
        w = max(nblk) if nblk else 0
        if width is not None:
            if w > width:
                raise RuntimeError(f"decode graph block table width {width} is smaller than runtime width {w}")
            w = width
        mirror = self._ensure_mirror(1 if tentative else 0)
        total = int(sum(qlens))
        pending = self._pending
        self._pending = {}
        if tentative:
            pending = {**pending, **tentative}
        n_up = len(pending)
        n_tok = total if token_ids is not None else 0
        arr = np.empty(5 * b + 3 * n_up + n_tok, dtype=np.int32)
        arr[0:b] = [self._row_of[s] for s in slots]
        arr[b:2 * b] = starts
        arr[2 * b:3 * b] = qlens
        arr[3 * b:4 * b] = nblk
        arr[4 * b:5 * b] = ctx
        if n_up:
            upd = arr[5 * b:5 * b + 3 * n_up].reshape(n_up, 3)
            upd[:, :2] = np.fromiter((x for rc in pending.keys() for x in rc), dtype=np.int32,
                                     count=2 * n_up).reshape(n_up, 2)
            upd[:, 2] = np.fromiter(pending.values(), dtype=np.int32, count=n_up)
        if n_tok:
            if isinstance(token_ids, np.ndarray):
                arr[5 * b + 3 * n_up:] = token_ids
            else:
                arr[5 * b + 3 * n_up:] = np.concatenate([np.asarray(t, dtype=np.int64) for t in token_ids])
        if self._uploader is None:
            self._uploader = _Uploader(self.device)
        dev = self._uploader.upload(arr)
        desc = dev[: 5 * b]
        upd_dev = dev[5 * b: 5 * b + 3 * n_up] if n_up else None
        tok_dev = dev[5 * b + 3 * n_up: 5 * b + 3 * n_up + n_tok] if n_tok else None

        def buf(name, shape, dtype):
            if out is not None and name in out:
                return out[name]
            return torch.empty(shape, dtype=dtype, device=self.device)

        block_tables = buf("block_tables", (b, w), torch.int32)
        context_lens = buf("context_lens", (b,), torch.int32)
        slot_mapping = buf("slot_mapping", (total,), torch.int64)
        positions = buf("positions", (total,), torch.int64)
        cu = buf("cu_seqlens_q", (b + 1,), torch.int32)
        last = buf("last_token_indices", (b,), torch.int64)
        input_ids = buf("input_ids", (total,), torch.int64) if n_tok else None
        _C.pack_batch(desc, b, upd_dev, n_up, tok_dev, mirror, bs, block_tables=block_tables,
                      context_lens=context_lens, slot_mapping=slot_mapping, positions=positions,
                      cu_seqlens=cu, last_token_indices=last, input_ids=input_ids)
        return PagedKVCacheMetadata(
            block_tables=block_tables, context_lens=context_lens, slot_mapping=slot_mapping,
            cu_seqlens_q=cu, positions=positions, last_token_indices=last, input_ids=input_ids,
            context_lens_host=ctx, max_context_len=max(ctx) if ctx else 0,
            max_query_len=max(qlens) if len(qlens) else 0,
        )

    def get_block_tables_tensor(self, slots: list[int]) -> torch.Tensor:
        return self._pack(slots, [0] * len(slots), [0] * len(slots)).block_tables

    def get_context_lens_tensor(self, slots: list[int]) -> torch.Tensor:
        """Device int32 [B] (the reference returns it on the host)."""
        return self._pack(slots, [0] * len(slots), [0] * len(slots)).context_lens

    def get_slot_mapping(self, slots: list[int], start_positions: list[int],
                         num_tokens_per_seq: list[int]) -> torch.Tensor:
        return self._pack(slots, list(start_positions), list(num_tokens_per_seq)).slot_mapping

    def prepare_prefill_metadata(self, slots: list[int], seq_lens: list[int], start_positions: list[int],
                                 prefix_block_ids: list[list[int]], token_ids=None) -> PagedKVCacheMetadata:
        if not (len(slots) == len(seq_lens) == len(start_positions) == len(prefix_block_ids)):
            raise ValueError("slots, seq_lens, start_positions and prefix_block_ids length mismatch")
        q_cum, kv_cum, tq, tkv = [], [], 0, 0
        for slot, n, start, prefix in zip(slots, seq_lens, start_positions, prefix_block_ids):
            self._init_slot(slot, start, prefix)
            end = start + n
            self.ensure_blocks(slot, end)
            self.seq_lens[slot] = max(self.seq_lens[slot], end)
            tq += n
            tkv += end
            q_cum.append(tq)
            kv_cum.append(tkv)
        md = self._pack(slots, list(start_positions), list(seq_lens), token_ids=token_ids)
        md.actual_seq_lengths_q = q_cum
        md.actual_seq_lengths_kv = kv_cum
        md.query_lens = list(seq_lens)
        md.use_paged_prefill = any(p > 0 for p in start_positions)
        return md

    def prepare_decode_metadata(self, slots: list[int], start_positions: list[int], q_len: int,
                                token_ids=None, width: int | None = None, out=None) -> PagedKVCacheMetadata:
        if len(slots) != len(start_positions):
            raise ValueError("slots and start_positions length mismatch")
        for slot, start in zip(slots, start_positions):
            end = start + q_len
            self.ensure_blocks(slot, end)
            if end > self.seq_lens[slot]:
                self.seq_lens[slot] = end
        return self._pack(slots, list(start_positions), [q_len] * len(slots), token_ids=token_ids, width=width,
                          out=out)

    # ------------------------------------------------ decode packed ahead of time
    def peek_decode_blocks(self, slots: list[int], start_positions: list[int],
                           q_len: int = 1) -> list[tuple[int, int]] | None:
        """The blocks ``prepare_decode_metadata(slots, start_positions, q_len)`` would allocate,
        as (slot, block id) in allocation order, without allocating them.

        None when such a step must not be packed ahead of its confirmation: the pool would run
        dry (the real call raises), or a block it would take still carries a prefix-cache key
        (a tentative write into it could corrupt content a later prefix hit reads).
        """
        want = []
        for slot, start in zip(slots, start_positions):
            have = len(self.block_tables[slot])
            want.extend([slot] * max(0, self._num_required_blocks(start + q_len) - have))
        if len(want) > len(self._free):
            return None
        taken = []
        for slot, block_id in zip(want, self._free):
            if self.blocks[block_id].block_hash is not None:
                return None
            taken.append((slot, block_id))
        return taken

    def prepare_decode_ahead(self, slots: list[int], start_positions: list[int], token_ids=None,
                             width: int | None = None, out=None):
        """Pack a one-token decode step whose batch is not confirmed yet.

        The step's metadata is exactly what ``prepare_decode_metadata`` will produce if nothing
        touches the pool before it is called with the same batch: its new blocks are the front
        of the free queue in batch order (``peek_decode_blocks``).  The pool, the tables and the
        context lengths are left unchanged; ``commit_decode_ahead`` applies the step once it is
        confirmed, and an unconfirmed step is simply forgotten.  Returns (metadata, taken), or
        None when the step cannot be packed ahead (see ``peek_decode_blocks``, or a graph width
        the step would outgrow).
        """
        if len(slots) != len(start_positions):
            raise ValueError("slots and start_positions length mismatch")
        taken = self.peek_decode_blocks(slots, start_positions, 1)
        if taken is None:
            return None
        tentative: dict[tuple[int, int], int] = {}
        for slot, block_id in taken:
            row = self._row_of[slot]
            col = len(self.block_tables[slot]) + sum(1 for (r, _) in tentative if r == row)
            tentative[(row, col)] = block_id
        if any(col > 0 and (r, col - 1) in tentative for (r, col) in tentative):
            return None  # two new blocks for one sequence: only one-token steps are packed ahead
        if width is not None and any(col >= width for (_, col) in tentative):
            return None
        if width is not None and any(len(self.block_tables[s]) > width for s in slots):
            return None
        md = self._pack(slots, list(start_positions), [1] * len(slots), token_ids=token_ids, width=width,
                        out=out, tentative=tentative)
        return md, taken

    def commit_decode_ahead(self, slots: list[int], start_positions: list[int],
                            taken: list[tuple[int, int]]) -> None:
        """Apply a confirmed step packed by ``prepare_decode_ahead``: allocate as
        ``prepare_decode_metadata`` does (same order, so the same blocks) and check that."""
        before = {slot: len(self.block_tables[slot]) for slot, _ in taken}
        for slot, start in zip(slots, start_positions):
            end = start + 1
            self.ensure_blocks(slot, end)
            if end > self.seq_lens[slot]:
                self.seq_lens[slot] = end
        got = [(slot, self.block_tables[slot][before[slot]]) for slot, _ in taken]
        if got != list(taken):
            raise RuntimeError(f"decode step packed ahead used blocks {taken}, the pool handed out {got}")
