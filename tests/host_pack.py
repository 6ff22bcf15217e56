"""CPU test double of the product BlockManager: metadata from the host state.

The allocation state machine is the product's, untouched; only ``_pack`` (the
GPU packing kernel) is replaced by the closed form
slot = table[pos // bs] * bs + pos % bs on the host.  It honours the same
arguments as the product's ``_pack``: a static ``width``, ``out`` buffers
(filled in place, zero-padded like a graph's static block table) and
``tentative`` blocks of a decode step packed ahead of its confirmation.
GPU packing itself is checked bit-exactly in test_pack_gpu.py.
"""
from __future__ import annotations

import torch

from nano_vllm_ascend_amd.block_manager import BlockManager, PagedKVCacheMetadata


class HostPackedBlockManager(BlockManager):
    def _pack(self, slots, starts, qlens, token_ids=None, width=None, out=None, tentative=None):
        bs = self.block_size
        tables = {s: list(self.block_tables[s]) for s in slots}
        for (row, col), block in (tentative or {}).items():
            slot = next(s for s in slots if self._row_of[s] == row)
            assert len(tables[slot]) == col, "a tentative block must extend its table"
            tables[slot].append(block)
        nblk = [len(tables[s]) for s in slots]
        w = max(nblk, default=0)
        if width is not None:
            if w > width:
                raise RuntimeError(f"decode graph block table width {width} is smaller than runtime width {w}")
            w = width
        bt = torch.zeros((len(slots), w), dtype=torch.int32)
        for i, s in enumerate(slots):
            bt[i, : nblk[i]] = torch.tensor(tables[s], dtype=torch.int32)
        sm, pos = [], []
        for s, st, n in zip(slots, starts, qlens):
            for p in range(st, st + n):
                if p // bs >= len(tables[s]):
                    raise RuntimeError(f"missing block: slot={s}, logical_pos={p}")
                sm.append(tables[s][p // bs] * bs + p % bs)
                pos.append(p)
        ctx = [max(self.seq_lens[s], st + n) for s, st, n in zip(slots, starts, qlens)]
        cu = [0]
        for n in qlens:
            cu.append(cu[-1] + n)
        ids = None
        if token_ids is not None:
            ids = torch.cat([torch.as_tensor(t, dtype=torch.int64).reshape(-1) for t in token_ids]) \
                if isinstance(token_ids, list) else torch.as_tensor(token_ids, dtype=torch.int64)
        md = PagedKVCacheMetadata(
            block_tables=bt, context_lens=torch.tensor(ctx, dtype=torch.int32),
            slot_mapping=torch.tensor(sm, dtype=torch.int64), cu_seqlens_q=torch.tensor(cu, dtype=torch.int32),
            positions=torch.tensor(pos, dtype=torch.int64),
            last_token_indices=torch.tensor(cu[1:], dtype=torch.int64) - 1, input_ids=ids,
            context_lens_host=ctx, max_context_len=max(ctx, default=0), max_query_len=max(qlens, default=0))
        if out is not None:
            for name in ("block_tables", "context_lens", "slot_mapping", "positions", "cu_seqlens_q",
                         "last_token_indices", "input_ids"):
                src = getattr(md, name)
                if name in out and src is not None:
                    out[name].copy_(src)
                    setattr(md, name, out[name])
        return md
