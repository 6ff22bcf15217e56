"""GPU packing (nvamd_pack_batch) is bit-exact with the reference block manager."""
from __future__ import annotations

import json
import random
import sys
from collections import OrderedDict
from pathlib import Path

import numpy as np
import pytest
import torch

from nano_vllm_ascend_amd import workloads as W
from nano_vllm_ascend_amd.block_manager import BlockManager
from nano_vllm_ascend_amd.engine import EngineCore
from nano_vllm_ascend_amd.sampling_params import SamplingParams
from nano_vllm_ascend_amd.scheduler import MiniScheduler
from nano_vllm_ascend_amd.sequence import Sequence
from oracle.block_manager_ref import BlockManagerRef

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import trace_driver  # noqa: E402


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(trace_driver.SCENARIOS))
def test_golden_trace_on_gpu(name, device):
    golden = json.loads((GOLDEN / "block_traces.json").read_text())[name]
    got = trace_driver.run_scenario(
        name, BlockManager=BlockManager, MiniScheduler=MiniScheduler, EngineCore=EngineCore, Sequence=Sequence,
        SamplingParams=SamplingParams, torch_mod=torch, device=device)
    got = json.loads(json.dumps(got))
    assert len(got) == len(golden)
    for i, (g, r) in enumerate(zip(got, golden)):
        assert g == r, f"{name}: event {i} differs\n got {g}\n ref {r}"


def _seeded_pair(num_blocks, block_size, seed, device, **kw):
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    ref = BlockManagerRef(num_blocks, block_size)
    ref.free_block_ids = list(perm)
    bm = BlockManager(num_blocks=num_blocks, block_size=block_size, device=device, **kw)
    bm._free = OrderedDict.fromkeys(perm)
    return ref, bm


@pytest.mark.gpu
def test_ragged_prefill_packing_32_prompts(device):
    """32 prompts of U[64, 2048] tokens, block_size 128, seeded free list of 1024 blocks."""
    lens = W.prefill_lengths(32, 64, 2048, seed=0)
    ref, bm = _seeded_pair(1024, 128, seed=0, device=device)
    rng = random.Random(0)
    tokens = [[rng.randint(0, 151935) for _ in range(n)] for n in lens]
    slots = list(range(32))
    a = ref.prepare_prefill_metadata(slots, lens, [0] * 32, [[] for _ in slots])
    b = bm.prepare_prefill_metadata(slots, lens, [0] * 32, [[] for _ in slots], token_ids=tokens)
    torch.cuda.synchronize()
    assert torch.equal(b.slot_mapping.cpu(), a.slot_mapping)
    assert torch.equal(b.block_tables.cpu(), a.block_tables)
    assert torch.equal(b.context_lens.cpu(), a.context_lens)
    assert b.actual_seq_lengths_q == a.actual_seq_lengths_q and b.actual_seq_lengths_kv == a.actual_seq_lengths_kv
    cu = [0] + a.actual_seq_lengths_q
    assert b.cu_seqlens_q.cpu().tolist() == cu
    assert b.last_token_indices.cpu().tolist() == [x - 1 for x in cu[1:]]
    assert b.positions.cpu().tolist() == [p for n in lens for p in range(n)]
    assert b.input_ids.cpu().tolist() == [t for seq in tokens for t in seq]


@pytest.mark.gpu
def test_packing_at_scale_small_blocks(device):
    """256 prompts of U[1, 4096] tokens in 16-token blocks (tables up to 256 entries wide) from a
    seeded free list, then 20 decode steps at batch 256: every step's slot mapping, tables and
    context lengths equal the oracle block manager's."""
    rng = random.Random(5)
    lens = [rng.randint(1, 4096) for _ in range(256)]
    num_blocks = sum((n + 20 + 15) // 16 for n in lens) + 64
    ref, bm = _seeded_pair(num_blocks, 16, seed=5, device=device, max_seqs=256)
    slots = list(range(256))

    def same(a, b, step):
        torch.cuda.synchronize()
        w = a.block_tables.shape[1]
        got = b.block_tables.cpu()
        assert torch.equal(got[:, :w], a.block_tables), step
        assert not got[:, w:].any(), step
        assert torch.equal(b.slot_mapping.cpu(), a.slot_mapping), step
        assert torch.equal(b.context_lens.cpu(), a.context_lens), step

    same(ref.prepare_prefill_metadata(slots, lens, [0] * 256, [[] for _ in slots]),
         bm.prepare_prefill_metadata(slots, lens, [0] * 256, [[] for _ in slots]), "prefill")
    pos = list(lens)
    for step in range(20):
        same(ref.prepare_decode_metadata(slots, pos, 1), bm.prepare_decode_metadata(slots, pos, 1), step)
        pos = [p + 1 for p in pos]


@pytest.mark.gpu
def test_decode_packing_into_static_graph_buffers(device):
    """Decode steps packed into fixed-width buffers; new blocks appear at page boundaries."""
    ref, bm = _seeded_pair(256, 16, seed=3, device=device, max_seqs=2, max_blocks_per_seq=2)
    lens = [5, 16, 31, 32, 47]
    slots = [10, 11, 12, 13, 14]
    ref.prepare_prefill_metadata(slots, lens, [0] * 5, [[] for _ in slots])
    bm.prepare_prefill_metadata(slots, lens, [0] * 5, [[] for _ in slots])
    width = 8
    out = {
        "block_tables": torch.full((5, width), -7, dtype=torch.int32, device=device),
        "context_lens": torch.empty(5, dtype=torch.int32, device=device),
        "slot_mapping": torch.empty(5, dtype=torch.int64, device=device),
        "positions": torch.empty(5, dtype=torch.int64, device=device),
        "input_ids": torch.empty(5, dtype=torch.int64, device=device),
    }
    pos = list(lens)
    for step in range(40):
        toks = [[1000 * step + i] for i in range(5)]
        a = ref.prepare_decode_metadata(slots, pos, 1)
        b = bm.prepare_decode_metadata(slots, pos, 1, token_ids=toks, width=width, out=out)
        torch.cuda.synchronize()
        assert b.block_tables is out["block_tables"]
        padded = torch.zeros((5, width), dtype=torch.int32)
        padded[:, : a.block_tables.shape[1]] = a.block_tables
        assert torch.equal(out["block_tables"].cpu(), padded), f"step {step}"
        assert torch.equal(out["slot_mapping"].cpu(), a.slot_mapping)
        assert torch.equal(out["context_lens"].cpu(), a.context_lens)
        assert out["positions"].cpu().tolist() == pos
        assert out["input_ids"].cpu().tolist() == [t[0] for t in toks]
        pos = [p + 1 for p in pos]
        if step == 17:  # a sequence leaves; its mirror row is recycled by a newcomer
            ref.free_slot(12)
            bm.free_slot(12)
            ref.prepare_prefill_metadata([15], [9], [0], [[]])
            bm.prepare_prefill_metadata([15], [9], [0], [[]])
            slots[2] = 15
            pos[2] = 9
    with pytest.raises(RuntimeError):
        bm.prepare_decode_metadata(slots, [p + 200 for p in pos], 1, width=width, out=out)


@pytest.mark.gpu
def test_prefix_hit_prefill_packing(device):
    """Retained prefix blocks appear in the tables; only the suffix gets slots."""
    ref, bm = _seeded_pair(64, 8, seed=5, device=device)
    toks = list(range(100, 140))
    for m in (ref, bm):
        m.prepare_prefill_metadata([0], [40], [0], [[]])
        m.cache_full_blocks(0, toks, 0, 5)
        m.free_slot(0)
    prefix_a = ref.find_longest_prefix_blocks(toks + [1, 2, 3], 5)
    prefix_b = bm.find_longest_prefix_blocks(toks + [1, 2, 3], 5)
    assert prefix_a == prefix_b and len(prefix_a) == 5
    a = ref.prepare_prefill_metadata([1, 2], [3, 7], [40, 0], [prefix_a, []])
    b = bm.prepare_prefill_metadata([1, 2], [3, 7], [40, 0], [prefix_b, []])
    torch.cuda.synchronize()
    assert b.use_paged_prefill and a.use_paged_prefill
    assert torch.equal(b.block_tables.cpu(), a.block_tables)
    assert torch.equal(b.slot_mapping.cpu(), a.slot_mapping)
    assert b.positions.cpu().tolist() == [40, 41, 42] + list(range(7))


@pytest.mark.gpu
def test_decode_step_packed_ahead_equals_the_confirmed_step(device):
    """A decode step packed ahead of its confirmation (GPU packing with tentative blocks for the
    sequences that open a block) equals, bit for bit, the metadata prepare_decode_metadata packs
    for the same step after the confirmation, and leaves the pool untouched until then."""
    rng = random.Random(7)
    ref, bm = _seeded_pair(256, 128, seed=7, device=device)
    lens = [127, 128, 129, 255, 256, 300, 511, 1, 64, 383]  # several open a block at the next position
    slots = list(range(len(lens)))
    bm.prepare_prefill_metadata(slots, lens, [0] * len(lens), [[] for _ in slots])
    ref.prepare_prefill_metadata(slots, lens, [0] * len(lens), [[] for _ in slots])
    width = 8
    for step in range(3):
        pos = [n + step for n in lens]
        bufs = {k: torch.full((len(slots), width) if k == "block_tables" else (len(slots) + (k == "cu_seqlens_q"),),
                              -7, dtype=torch.int32 if k in ("block_tables", "context_lens", "cu_seqlens_q")
                              else torch.int64, device=device)
                for k in ("block_tables", "context_lens", "slot_mapping", "positions", "cu_seqlens_q",
                          "last_token_indices", "input_ids")}
        free_before = list(bm.free_block_ids)
        toks = np.array([rng.randint(0, 1000) for _ in slots], dtype=np.int64)
        md, taken = bm.prepare_decode_ahead(slots, pos, token_ids=toks, width=width, out=bufs)
        torch.cuda.synchronize()
        got = {k: v.cpu().clone() for k, v in bufs.items()}
        assert bm.free_block_ids == free_before
        bm.commit_decode_ahead(slots, pos, taken)
        want = bm.prepare_decode_metadata(slots, pos, 1, token_ids=toks, width=width)
        r = ref.prepare_decode_metadata(slots, pos, 1)
        torch.cuda.synchronize()
        assert torch.equal(got["block_tables"], want.block_tables.cpu())
        assert torch.equal(got["block_tables"][:, : r.block_tables.shape[1]], r.block_tables)
        for k, attr in (("context_lens", "context_lens"), ("slot_mapping", "slot_mapping"),
                        ("positions", "positions"), ("input_ids", "input_ids")):
            assert torch.equal(got[k], getattr(want, attr).cpu()), (step, k)
        assert torch.equal(got["context_lens"], r.context_lens) and torch.equal(got["slot_mapping"], r.slot_mapping)
        assert got["context_lens"].tolist() == [p + 1 for p in pos]
        # step 0 writes positions 128 and 256 into new blocks; step 1 positions 128, 256, 384, 512
        assert len(taken) == {0: 2, 1: 4, 2: 0}[step]
