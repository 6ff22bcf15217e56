"""Block manager: the reference's known answers, golden traces and state-machine equivalence (CPU).

The product BlockManager builds its metadata tensors on the GPU; on the CPU
these tests check its allocation state machine through a test-only subclass
that derives the metadata from the host state with the closed form
slot = table[pos // bs] * bs + pos % bs.  GPU packing itself is checked
bit-exactly in test_pack_gpu.py.
"""
from __future__ import annotations

import json
import random
import sys
from pathlib import Path

import pytest
import torch

from nano_vllm_ascend_amd.engine import EngineCore
from nano_vllm_ascend_amd.sampling_params import SamplingParams
from nano_vllm_ascend_amd.scheduler import MiniScheduler
from nano_vllm_ascend_amd.sequence import Sequence
from oracle.block_manager_ref import BlockManagerRef

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import trace_driver  # noqa: E402
from host_pack import HostPackedBlockManager  # noqa: E402


MANAGERS = [BlockManagerRef, HostPackedBlockManager]


def make(cls, num_blocks=8, block_size=4):
    if cls is BlockManagerRef:
        return cls(num_blocks, block_size)
    return cls(num_blocks=num_blocks, block_size=block_size, device="cpu")


# --- the reference's known answers (tests/test_block_manager.py:6-54) ---
@pytest.mark.parametrize("cls", MANAGERS)
def test_prefill_metadata_cumulative_lengths_and_slots(cls):
    bm = make(cls)
    md = bm.prepare_prefill_metadata(slots=[0, 1, 2], seq_lens=[3, 5, 2], start_positions=[0, 0, 0],
                                     prefix_block_ids=[[], [], []])
    assert md.actual_seq_lengths_q == [3, 8, 10]
    assert md.actual_seq_lengths_kv == [3, 8, 10]
    assert md.context_lens.tolist() == [3, 5, 2]
    assert md.slot_mapping.tolist() == [0, 1, 2, 4, 5, 6, 7, 8, 12, 13]
    assert md.block_tables.tolist() == [[0, 0], [1, 2], [3, 0]]


@pytest.mark.parametrize("cls", MANAGERS)
def test_decode_metadata_for_active_slots_and_positions(cls):
    bm = make(cls)
    bm.prepare_prefill_metadata(slots=[0, 1, 2], seq_lens=[3, 5, 2], start_positions=[0, 0, 0],
                                prefix_block_ids=[[], [], []])
    md = bm.prepare_decode_metadata(slots=[1, 2], start_positions=[5, 2], q_len=1)
    assert md.context_lens.tolist() == [6, 3]
    assert md.slot_mapping.tolist() == [9, 14]


@pytest.mark.parametrize("cls", MANAGERS)
def test_prefix_cache_reuses_full_blocks(cls):
    bm = make(cls)
    tokens = torch.tensor([10, 11, 12, 13, 20, 21], dtype=torch.long)
    bm.prepare_prefill_metadata(slots=[0], seq_lens=[6], start_positions=[0], prefix_block_ids=[[]])
    bm.cache_full_blocks(slot=0, token_ids=tokens)
    bm.free_slot(0)
    assert bm.find_longest_prefix_blocks(tokens, max_cache_blocks=1) == [0]


@pytest.mark.parametrize("cls", MANAGERS)
def test_errors_follow_reference(cls):
    bm = make(cls, num_blocks=2, block_size=4)
    with pytest.raises(ValueError):
        bm.prepare_prefill_metadata(slots=[0], seq_lens=[1, 2], start_positions=[0], prefix_block_ids=[[]])
    with pytest.raises(RuntimeError):
        bm.prepare_prefill_metadata(slots=[0], seq_lens=[9], start_positions=[0], prefix_block_ids=[[]])
    bm2 = make(cls, num_blocks=4, block_size=4)
    bm2.prepare_prefill_metadata(slots=[0], seq_lens=[3], start_positions=[0], prefix_block_ids=[[]])
    bm2.free_slot(0)
    with pytest.raises(RuntimeError):
        bm2._release_block(0)
    bm2.prepare_prefill_metadata(slots=[1], seq_lens=[3], start_positions=[0], prefix_block_ids=[[]])
    with pytest.raises(RuntimeError):
        bm2.clear_prefix_cache()


# --- golden traces written from the reference source ---
def _replay(name, cls):
    return trace_driver.run_scenario(
        name, BlockManager=lambda num_blocks, block_size, device: make(cls, num_blocks, block_size),
        MiniScheduler=MiniScheduler, EngineCore=EngineCore, Sequence=Sequence, SamplingParams=SamplingParams,
        torch_mod=torch)


@pytest.mark.parametrize("cls", MANAGERS)
@pytest.mark.parametrize("name", sorted(trace_driver.SCENARIOS))
def test_golden_trace(name, cls):
    golden = json.loads((GOLDEN / "block_traces.json").read_text())[name]
    got = json.loads(json.dumps(_replay(name, cls)))
    assert len(got) == len(golden)
    for i, (g, r) in enumerate(zip(got, golden)):
        assert g == r, f"{name}: event {i} differs\n got {g}\n ref {r}"


# --- randomized equivalence of the two state machines ---
@pytest.mark.parametrize("seed", range(6))
def test_state_machine_matches_oracle_on_random_ops(seed):
    rng = random.Random(seed)
    bs, nb = 4, 32
    ref = BlockManagerRef(nb, bs)
    got = HostPackedBlockManager(num_blocks=nb, block_size=bs, device="cpu")
    live: dict[int, list[int]] = {}
    next_slot = 0
    vocab = [rng.randint(0, 5) for _ in range(64)]
    for _ in range(300):
        op = rng.random()
        if op < 0.35 and len(live) < 6:
            n = rng.randint(1, 14)
            toks = [vocab[rng.randint(0, 8)] for _ in range(n)]
            max_blocks = n // bs - (1 if n % bs == 0 and n >= bs else 0)
            prefix = ref.find_longest_prefix_blocks(toks, max_blocks) if max_blocks > 0 else []
            assert prefix == (got.find_longest_prefix_blocks(toks, max_blocks) if max_blocks > 0 else [])
            start = len(prefix) * bs
            need = -(-(n + 2) // bs) - len(prefix)
            if need > len(ref.free_block_ids):
                continue
            a = ref.prepare_prefill_metadata([next_slot], [n - start], [start], [prefix])
            b = got.prepare_prefill_metadata([next_slot], [n - start], [start], [prefix])
            assert a.slot_mapping.tolist() == b.slot_mapping.tolist()
            ref.cache_full_blocks(next_slot, toks, len(prefix), n // bs)
            got.cache_full_blocks(next_slot, toks, len(prefix), n // bs)
            live[next_slot] = toks
            next_slot += 1
        elif op < 0.7 and live:
            slots = sorted(live)
            starts = [len(live[s]) for s in slots]
            total_new = sum(1 for s in slots if len(live[s]) % bs == 0)
            if total_new > len(ref.free_block_ids):
                continue
            a = ref.prepare_decode_metadata(slots, starts, 1)
            b = got.prepare_decode_metadata(slots, starts, 1)
            assert a.block_tables.tolist() == b.block_tables.tolist()
            assert a.slot_mapping.tolist() == b.slot_mapping.tolist()
            assert a.context_lens.tolist() == b.context_lens.tolist()
            for s in slots:
                live[s].append(rng.randint(0, 5))
        elif live:
            s = rng.choice(sorted(live))
            ref.free_slot(s)
            got.free_slot(s)
            del live[s]
        assert ref.free_block_ids == got.free_block_ids
        assert ref.block_tables == got.block_tables
        assert [b.ref_count for b in ref.blocks] == [b.ref_count for b in got.blocks]
        assert [b.block_hash is None for b in ref.blocks] == [b.block_hash is None for b in got.blocks]
