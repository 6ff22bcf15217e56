"""Overlapped decode on the GPU keeps the reference's packing metadata (real model, real kernels).

The product ``LLM`` (2-layer Qwen3-0.6B-shaped model, 128-token blocks, prefix
cache on, overlap on, decode graphs) runs a submission schedule with requests
admitted mid-run, a shared 2-block prefix and an EOS token that some requests
sample mid-run.  A metadata hook records the block tables, slot mappings and
context lengths of every prefill and of every decode step actually taken
(steps launched ahead and discarded are not).  The oracle engine and block
manager replay the same schedule with the tokens this run produced; every
step must match bit for bit.  Tokens must equal the synchronous loop's.
"""
from __future__ import annotations

import sys
from dataclasses import replace
from pathlib import Path

import pytest
import torch

from nano_vllm_ascend_amd import LLM
from nano_vllm_ascend_amd.config import QWEN3_0_6B

sys.path.insert(0, str(Path(__file__).resolve().parent))
from trace_check import assert_same_metadata, make_schedule, oracle_replay, run_product  # noqa: E402

SMALL = replace(QWEN3_0_6B, num_hidden_layers=2)
CFG = dict(block_size=128, num_blocks=30, max_num_seqs=4, prefix=True)


def make(overlap: bool) -> LLM:
    return LLM(SMALL, max_model_len=1024, block_size=CFG["block_size"], num_blocks=CFG["num_blocks"],
               max_num_seqs=CFG["max_num_seqs"], enable_prefix_cache=CFG["prefix"], enable_decode_graph=True,
               seed=1, enable_overlap=overlap)


@pytest.mark.gpu
def test_overlapped_engine_metadata_equals_oracle_replay(device):
    schedule = make_schedule(seed=31, n=10, block_size=128, len_lo=60, len_hi=260, new_lo=10, new_hi=150,
                             shared_blocks=2)
    _, plain, _ = run_product(make(False), schedule, -1)
    # an EOS token the model samples mid-run in request 1 (and wherever else it appears)
    eos = plain[1][len(plain[1]) // 2]
    print(f"[overlap trace] eos token {eos}", flush=True)
    sync_events, sync_out, sync_reasons = run_product(make(False), schedule, eos)
    llm = make(True)
    events, out, reasons = run_product(llm, schedule, eos)
    stats = dict(llm.runner.overlap_stats)
    print(f"[overlap trace] {stats}; finish reasons {sorted(reasons.items())}; "
          f"graph {llm.runner.decode_graph_stats()}", flush=True)
    assert out == sync_out and reasons == sync_reasons
    assert "eos" in reasons.values()
    assert stats["launched"] > 0 and stats["used"] > 0
    ref = oracle_replay(schedule, out, reasons, eos, **CFG)
    assert_same_metadata(sync_events, ref)
    assert_same_metadata(events, ref)
    del llm
    torch.cuda.empty_cache()


@pytest.mark.gpu
@pytest.mark.parametrize("seed,bs,blocks,seqs,prefix", [(41, 128, 60, 8, True), (42, 64, 90, 6, False),
                                                        (43, 16, 400, 8, True)])
def test_random_schedules_metadata_equals_oracle_replay(device, seed, bs, blocks, seqs, prefix):
    """Seeded schedules of 12 requests (prompts of 20-300 tokens behind a shared 2-block prefix on
    even requests when the cache is on, 5-120 new tokens, half admitted mid-run), block sizes 128,
    64 and 16, up to 8 running sequences (decode graphs of 1-8 rows), overlapped decode, an EOS the
    model samples mid-run: every prefill and decode step's metadata equals the oracle engine's
    replay of the same run."""
    schedule = make_schedule(seed=seed, n=12, block_size=bs, len_lo=20, len_hi=300, new_lo=5, new_hi=120,
                             shared_blocks=2 if prefix else 0)

    def build():
        return LLM(SMALL, max_model_len=1024, block_size=bs, num_blocks=blocks, max_num_seqs=seqs,
                   enable_prefix_cache=prefix, enable_decode_graph=True, seed=seed, enable_overlap=True)

    _, plain, _ = run_product(build(), schedule, -1)
    longest = max(plain, key=lambda i: len(plain[i]))
    eos = plain[longest][len(plain[longest]) // 2]
    llm = build()
    events, out, reasons = run_product(llm, schedule, eos)
    print(f"[random schedule {seed}] bs {bs}: {len(events)} steps, overlap {dict(llm.runner.overlap_stats)}, "
          f"finish reasons {sorted(set(reasons.values()))}", flush=True)
    assert "eos" in reasons.values()
    ref = oracle_replay(schedule, out, reasons, eos, block_size=bs, num_blocks=blocks, max_num_seqs=seqs,
                        prefix=prefix)
    assert_same_metadata(events, ref)
    del llm
    torch.cuda.empty_cache()
