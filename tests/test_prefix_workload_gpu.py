"""The 100 x 2048 load workload with a shared prefix really shares KV pages (2-layer model, short output).

Reference semantics (nv/model_runner.py:146-167, 232-238): the prefix lookup happens when a
request is submitted and blocks are cached only after their prefill, so a seed request that
carries the shared prefix is run first.  Then all 100 requests are submitted: the 50 that share
the 1024-token prefix must each hold the same 8 cached blocks (every one of them referenced 50
times while they run), the batch's prefill must take the paged route, the batch-100 decode graph
must be captured and replayed, and the tokens must equal a run without the prefix cache (a row
may differ only at a near-tie, after which it leaves the comparison).
"""
from __future__ import annotations

from dataclasses import replace

import pytest
import torch

from nano_vllm_ascend_amd import LLM
from nano_vllm_ascend_amd.bench_e2e import make_dataset
from nano_vllm_ascend_amd.config import QWEN3_0_6B

SMALL = replace(QWEN3_0_6B, num_hidden_layers=2)
N, PROMPT, SHARED, NEW = 100, 2048, 1024, 8
TIE_TOL = 0.05


def make(prefix: bool) -> LLM:
    llm = LLM(SMALL, max_model_len=4096, block_size=128, num_blocks=N * 17 + 32, max_num_seqs=N,
              enable_prefix_cache=prefix, decode_graph_batch_sizes=[1, 2, 4, 8, 16, 32, 64, 100], seed=1,
              retain_logits=True)
    llm.runner.tokenizer.eos_token_id = -1
    return llm


@pytest.mark.gpu
def test_shared_prefix_workload_hits_the_cache_and_matches_no_cache(device):
    prompts = make_dataset(N, PROMPT, SMALL.vocab_size, seed=0, shared_prefix=SHARED, shared_fraction=0.5)
    assert all(p[:SHARED] == prompts[0][:SHARED] for p in prompts[: N // 2])
    cached, plain = make(True), make(False)
    cached.generate([prompts[0][:SHARED] + [7]], max_new_tokens=1)  # the seed request caches 8 blocks
    assert cached.runner.prefill_stats["paged_batches"] == 0
    for llm in (cached, plain):
        llm.scheduler.reset()
        for p in prompts:
            llm.submit(p, max_new_tokens=NEW)
    seqs = cached.scheduler.seqs
    hit = [len(seqs[i].cached_block_ids) for i in range(N)]
    assert hit == [SHARED // 128] * (N // 2) + [0] * (N // 2)
    prefix_blocks = seqs[0].cached_block_ids
    assert all(seqs[i].cached_block_ids == prefix_blocks for i in range(N // 2))

    live, dropped, step = set(range(N)), 0, 0
    while cached.has_unfinished():
        cached.step()
        plain.step()
        if step == 0:  # after the prefill: each shared block is held by the 50 requests
            refs = [cached.runner.block_manager.blocks[b].ref_count for b in prefix_blocks]
            assert refs == [N // 2] * len(prefix_blocks), refs
        step += 1
        if not cached.has_unfinished():
            break
        lb = plain.runner.last_logits.float()
        ta = [s.next_token_id for s in cached.scheduler.seqs.values()]
        tb = [s.next_token_id for s in plain.scheduler.seqs.values()]
        for row in sorted(live):
            if ta[row] != tb[row]:
                assert (lb[row, tb[row]] - lb[row, ta[row]]).item() < TIE_TOL, (row, step)
                live.discard(row)
                dropped += 1
    got = {i: s.generated_token_ids for i, s in cached.scheduler.finished.items()}
    want = {i: s.generated_token_ids for i, s in plain.scheduler.finished.items()}
    same = sum(got[i] == want[i] for i in range(N))
    stats = cached.runner.prefill_stats
    graph = cached.runner.decode_graph_stats()
    print(f"[load workload] {same}/{N} requests token-equal to the no-cache run ({dropped} left at near-ties); "
          f"prefill {stats}; graph {graph}", flush=True)
    assert stats["paged_batches"] == 1 and stats["cached_tokens"] == (N // 2) * SHARED
    assert graph["captures"] >= 1 and graph["replays"] >= NEW - 2 and graph["capture_failures"] == 0
    assert same >= 0.9 * N
    del cached, plain
    torch.cuda.empty_cache()
