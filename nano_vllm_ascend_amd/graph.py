"""hipGraph replay of the decode forward (nv/npu/acl_graph.py:13-267).

One graph per exact decode batch size, captured the first time that size is
seen; a failed capture disables only that size and the caller falls back to
eager.  Static inputs per entry: input_ids, positions, a block table of fixed
width ceil(max_model_len / block_size), context_lens, slot_mapping, and the
paged-decode workspace.  The decode kernel reads context_lens from the
device, so a replay needs no host work besides filling the static inputs --
the reference re-issued all 28 paged-attention tasks from the host before
every replay.  ``DecodeGraphRunner.forward`` keeps the reference's
copy-then-replay call; the model runner instead packs the next step's
metadata straight into an entry's buffers (``entry_for`` + ``replay``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _C
from .block_manager import PagedKVCacheMetadata


class DecodeGraphStats:
    def __init__(self) -> None:
        self.captures = 0
        self.replays = 0
        self.updates = 0      # static-input refreshes (one per replay)
        self.fallbacks = 0
        self.capture_failures = 0

    def as_dict(self) -> dict[str, int]:
        return {"captures": self.captures, "replays": self.replays, "updates": self.updates,
                "fallbacks": self.fallbacks, "capture_failures": self.capture_failures}


def copy_block_tables(target: torch.Tensor, source: torch.Tensor) -> None:
    """Zero-padded copy of a [B, w] table into a [B, W] static one (W >= w)."""
    if source.shape[1] > target.shape[1]:
        raise RuntimeError(
            f"decode graph block table width {target.shape[1]} is smaller than runtime width {source.shape[1]}")
    target.zero_()
    target[:, : source.shape[1]].copy_(source)


@dataclass
class DecodeGraphEntry:
    batch_size: int
    width: int
    buffers: dict
    metadata: PagedKVCacheMetadata
    graph: object = None
    logits: torch.Tensor | None = None

    def copy_inputs(self, input_ids, position_ids, attn_metadata) -> None:
        b = self.buffers
        if attn_metadata is self.metadata:
            return  # already packed into the static buffers
        b["input_ids"].copy_(input_ids)
        b["positions"].copy_(position_ids)
        copy_block_tables(b["block_tables"], attn_metadata.block_tables)
        b["context_lens"].copy_(attn_metadata.context_lens)
        b["slot_mapping"].copy_(attn_metadata.slot_mapping)


class DecodeGraphRunner:
    def __init__(self, model, kv_cache, batch_sizes: list[int], max_model_len: int | None = None,
                 block_size: int | None = None):
        self.model = model
        self.kv_cache = kv_cache
        self.batch_sizes = set(batch_sizes)
        self.block_size = block_size
        self.max_blocks_per_seq = None
        if max_model_len is not None and block_size is not None:
            self.max_blocks_per_seq = math.ceil(max_model_len / block_size)
        self.entries: dict[int, DecodeGraphEntry] = {}
        self.disabled_batch_sizes: set[int] = set()
        self.stats = DecodeGraphStats()
        self._pool = None
        # graph primitives (replaceable by tests that run without a GPU)
        self.make_graph = torch.cuda.CUDAGraph
        self.graph_context = lambda g, pool: torch.cuda.graph(g, pool=pool)
        self.synchronize = torch.cuda.synchronize

    def supports(self, batch_size: int) -> bool:
        return batch_size in self.batch_sizes and batch_size not in self.disabled_batch_sizes

    def entry_for(self, batch_size: int, width_hint: int, device, block_size: int | None = None) -> DecodeGraphEntry:
        """The entry of a batch size (static buffers allocated on first use; captured lazily)."""
        entry = self.entries.get(batch_size)
        if entry is not None:
            return entry
        bs = block_size or self.block_size or self.kv_cache.block_size
        width = self.max_blocks_per_seq or width_hint
        b = batch_size
        bufs = {
            "input_ids": torch.zeros(b, dtype=torch.int64, device=device),
            "positions": torch.zeros(b, dtype=torch.int64, device=device),
            "block_tables": torch.zeros((b, width), dtype=torch.int32, device=device),
            "context_lens": torch.ones(b, dtype=torch.int32, device=device),
            "slot_mapping": torch.zeros(b, dtype=torch.int64, device=device),
            "cu_seqlens_q": torch.zeros(b + 1, dtype=torch.int32, device=device),
            "last_token_indices": torch.zeros(b, dtype=torch.int64, device=device),
        }
        # In-graph argmax of the logits, written over the input ids: the embedding has read them by
        # then, so a replay launched right behind this one takes this step's tokens as its inputs
        # without a copy (a host-packed step writes its own ids before its replay).
        bufs["greedy_ids"] = bufs["input_ids"]
        cfg = getattr(self.model, "config", None)
        hq = getattr(cfg, "num_attention_heads", 1)
        hkv = getattr(cfg, "num_key_value_heads", 1)
        md = PagedKVCacheMetadata(
            block_tables=bufs["block_tables"], context_lens=bufs["context_lens"], slot_mapping=bufs["slot_mapping"],
            cu_seqlens_q=bufs["cu_seqlens_q"], positions=bufs["positions"],
            last_token_indices=bufs["last_token_indices"], input_ids=bufs["input_ids"],
            max_context_bound=width * bs,
            decode_workspace=_C.alloc_paged_decode_workspace(b, hq, hkv, width * bs, device),
        )
        entry = DecodeGraphEntry(batch_size=b, width=width, buffers=bufs, metadata=md)
        self.entries[b] = entry
        return entry

    def _capture(self, entry: DecodeGraphEntry) -> bool:
        b = entry.buffers
        try:
            self.synchronize()
            # one eager run first: lazy library state is created outside the capture;
            # it writes the same KV slots the first replay writes
            self.model(input_ids_flat=b["input_ids"], position_ids_flat=b["positions"], kv_cache=self.kv_cache,
                       attn_metadata=entry.metadata, is_prefill=False)
            self.synchronize()
            graph = self.make_graph()
            with self.graph_context(graph, self._pool):
                out = self.model(input_ids_flat=b["input_ids"], position_ids_flat=b["positions"],
                                 kv_cache=self.kv_cache, attn_metadata=entry.metadata, is_prefill=False)
                if getattr(out.logits, "is_cuda", False):
                    _C.argmax_rows(out.logits, b["greedy_ids"])
            if self._pool is None and hasattr(graph, "pool"):
                self._pool = graph.pool()
            entry.graph = graph
            entry.logits = out.logits
        except Exception as exc:  # the reference disables the size and falls back (nv/npu/acl_graph.py:198-202)
            self.disabled_batch_sizes.add(entry.batch_size)
            self.entries.pop(entry.batch_size, None)
            self.stats.capture_failures += 1
            print(f"[decode_graph] disable batch_size={entry.batch_size}: {exc}")
            return False
        self.stats.captures += 1
        return True

    def replay(self, entry: DecodeGraphEntry) -> torch.Tensor | None:
        """Replay an entry whose static inputs are filled; capture on first use.  None if capture failed."""
        if entry.graph is None and not self._capture(entry):
            self.stats.fallbacks += 1
            return None
        self.stats.updates += 1
        entry.graph.replay()
        self.stats.replays += 1
        return entry.logits

    def forward(self, input_ids: torch.Tensor, position_ids: torch.Tensor,
                attn_metadata: PagedKVCacheMetadata) -> torch.Tensor | None:
        batch_size = int(input_ids.numel())
        if not self.supports(batch_size):
            self.stats.fallbacks += 1
            return None
        entry = self.entry_for(batch_size, attn_metadata.block_tables.shape[1], input_ids.device)
        entry.copy_inputs(input_ids, position_ids, attn_metadata)
        return self.replay(entry)

    def stats_dict(self) -> dict[str, int]:
        return self.stats.as_dict()
