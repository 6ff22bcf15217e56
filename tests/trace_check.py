"""Replaying a product run through the oracle engine, for the packing-order tests (CPU and GPU).

``run_product`` drives an ``LLM`` from a submission schedule with a metadata
hook on its runner; ``oracle_replay`` feeds the same schedule and the tokens
that run produced (EOS included) to the oracle engine and block manager
(oracle/engine_ref.py, oracle/block_manager_ref.py, pinned by the golden
traces); ``assert_same_metadata`` compares the two event streams bit for bit
(block tables up to the oracle's width, zero padding beyond it, slot mapping,
context lengths).
"""
from __future__ import annotations

import random
import sys
from pathlib import Path

import torch

from nano_vllm_ascend_amd.sampling_params import SamplingParams
from oracle.block_manager_ref import BlockManagerRef
from oracle.engine_ref import EngineRef, SchedulerRef, SequenceRef

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import trace_driver  # noqa: E402

ORACLE = dict(BlockManager=lambda num_blocks, block_size, device: BlockManagerRef(num_blocks, block_size),
              MiniScheduler=SchedulerRef, EngineCore=EngineRef, Sequence=SequenceRef, SamplingParams=SamplingParams,
              torch_mod=torch)


def make_schedule(seed, n, block_size, len_lo, len_hi, new_lo, new_hi, shared_blocks):
    rng = random.Random(seed)
    shared = [rng.randint(0, 400) for _ in range(shared_blocks * block_size)]
    schedule: dict[int, list] = {}
    for i in range(n):
        body = [rng.randint(0, 400) for _ in range(rng.randint(len_lo, len_hi))]
        step = 0 if i < n // 2 else 3 * (i - n // 2) + 1
        schedule.setdefault(step, []).append((shared + body if i % 2 == 0 else body, rng.randint(new_lo, new_hi)))
    return schedule


def run_product(llm, schedule, eos, events=None):
    llm.runner.tokenizer.eos_token_id = eos
    events = [] if events is None else events

    def hook(kind, slots, md):
        events.append({"event": kind, "slots": slots, "block_tables": md.block_tables.tolist(),
                       "context_lens": md.context_lens.tolist(), "slot_mapping": md.slot_mapping.tolist()})

    llm.runner.metadata_hook = hook
    finished, step = {}, 0
    while llm.has_unfinished() or step <= max(schedule):
        for tokens, max_new in schedule.get(step, []):
            llm.submit(tokens, max_new_tokens=max_new)
        for out in llm.step():
            finished[out["request_id"]] = out["token_ids"]
        step += 1
    reasons = {i: s.finish_reason for i, s in llm.scheduler.finished.items()}
    return events, finished, reasons


def oracle_replay(schedule, outputs, reasons, eos, *, block_size, num_blocks, max_num_seqs, prefix):
    def token_fn(seq_id, n):
        out = outputs[seq_id]
        if n < len(out):
            return out[n]
        assert reasons[seq_id] == "eos"
        return eos

    events = trace_driver.run_schedule(schedule, token_fn, eos, block_size=block_size, num_blocks=num_blocks,
                                       max_num_seqs=max_num_seqs, prefix_cache=prefix, **ORACLE)
    return [e for e in events if e["event"] in ("prefill", "decode")]


def assert_same_metadata(got, ref):
    assert len(got) == len(ref)
    for i, (g, r) in enumerate(zip(got, ref)):
        assert (g["event"], g["slots"]) == (r["event"], r["slots"]), i
        w = len(r["block_tables"][0]) if r["block_tables"] else 0
        assert [row[:w] for row in g["block_tables"]] == r["block_tables"], (i, g, r)
        assert all(x == 0 for row in g["block_tables"] for x in row[w:]), i  # zero padding of a static table
        assert g["slot_mapping"] == r["slot_mapping"], (i, g, r)
        assert g["context_lens"] == r["context_lens"], (i, g, r)
