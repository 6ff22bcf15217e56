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
