"""Parity of the load workload against the oracle: 100 requests x 2048 prompt tokens, half of them
sharing one 1024-token prefix, prefix cache on, decode graphs up to batch 100.

Three parts of that workload, each against the oracle on the same inputs:

* metadata -- the product engine (2-layer Qwen3-0.6B-shaped model, overlapped decode, as the bench
  runs it) takes a seed request carrying the prefix, then the 100 requests; every prefill and decode
  step it takes must carry the block tables, slot mapping and context lengths that the oracle engine
  and block manager produce when they replay the same schedule and tokens (nv/model_runner.py:146-167,
  232-238; nv/npu/block_manager.py:136-192, 252-328).  The decode runs long enough that every
  sequence opens two new blocks.
* paged prefill -- 100 x (1024 cached + 1024 new) for the sharing half and 2048 new for the rest, in
  one launch over pages where the sharing rows hold the same 8 physical blocks; 8 sequences (4 of
  each kind) against paged_prefill_ref, and every row against the dense prefill of its whole prompt
  (the reference's cache-hit == no-cache invariant, docs/prefix_cache_hit_analysis.md:195-207).
* decode -- 100 x U[2048, 4096] contexts, rows 0-49 sharing their first 8 blocks, plain and fused
  (norm + RoPE + KV store + attention), against paged_decode_ref and the composed oracle.
"""
from __future__ import annotations

import random
import sys
from dataclasses import replace
from pathlib import Path

import pytest
import torch

from nano_vllm_ascend_amd import LLM, _C
from nano_vllm_ascend_amd import workloads as W
from nano_vllm_ascend_amd.bench_e2e import make_dataset
from nano_vllm_ascend_amd.config import QWEN3_0_6B
from oracle.attention_ref import paged_decode_ref, paged_prefill_ref

sys.path.insert(0, str(Path(__file__).resolve().parent))
from test_fused_decode_gpu import Case  # noqa: E402
from trace_check import assert_same_metadata, oracle_replay, run_product  # noqa: E402

SMALL = replace(QWEN3_0_6B, num_hidden_layers=2)
N, PROMPT, SHARED, BS = 100, 2048, 1024, 128
NEW = 260  # 259 decode steps: positions 2048..2306 open blocks 16 and 17 (and 18 at 2304)
TOL = 2e-2
SCALE = 128 ** -0.5


def _schedule():
    prompts = make_dataset(N, PROMPT, SMALL.vocab_size, seed=0, shared_prefix=SHARED, shared_fraction=0.5)
    seed_prompt = prompts[0][:SHARED] + [prompts[N // 2][0]]  # as the bench's seed request
    return prompts, {0: [(seed_prompt, 1)], 3: [(p, NEW) for p in prompts]}


@pytest.mark.gpu
def test_load_workload_metadata_equals_oracle_replay(device):
    prompts, schedule = _schedule()
    cfg = dict(block_size=BS, num_blocks=N * 19 + 32, max_num_seqs=N, prefix=True)
    llm = LLM(SMALL, max_model_len=4096, block_size=BS, num_blocks=cfg["num_blocks"], max_num_seqs=N,
              enable_prefix_cache=True, decode_graph_batch_sizes=[1, 2, 4, 8, 16, 32, 64, 100], seed=1)
    events, out, reasons = run_product(llm, schedule, -1)
    seqs = {**llm.scheduler.finished}
    hits = [len(seqs[i].cached_block_ids) for i in range(1, N + 1)]
    stats, graph = dict(llm.runner.prefill_stats), llm.runner.decode_graph_stats()
    n_prefill = sum(e["event"] == "prefill" for e in events)
    n_decode = sum(e["event"] == "decode" for e in events)
    print(f"[load metadata] {n_prefill} prefill and {n_decode} decode steps; prefill {stats}; graph {graph}; "
          f"overlap {dict(llm.runner.overlap_stats)}", flush=True)
    assert hits == [SHARED // BS] * (N // 2) + [0] * (N // 2)
    assert stats["paged_batches"] == 1 and stats["cached_tokens"] == (N // 2) * SHARED
    assert graph["capture_failures"] == 0 and graph["replays"] >= NEW - 10
    assert n_decode >= NEW - 1
    ref = oracle_replay(schedule, out, reasons, -1, **cfg)
    assert_same_metadata(events, ref)
    # the last decode step still holds the whole batch, and every sequence opened its 17th, 18th and
    # 19th blocks in decode (contexts past 2048 + 2 * 128 tokens)
    last = [e for e in events if e["event"] == "decode"][-1]
    assert len(last["slots"]) == N
    assert min(last["context_lens"]) > PROMPT + 2 * BS
    del llm
    torch.cuda.empty_cache()


def _shared_tables(ctx, shared_rows, shared_blocks, seed, num_blocks=None):
    """Seeded block tables over a pool of `num_blocks` (default: just enough) in which rows
    [0, shared_rows) hold one physical copy of their first `shared_blocks` blocks (the prefix-cache
    hit); every other block is private."""
    need = [-(-c // BS) for c in ctx]
    least = shared_blocks + sum(n - (shared_blocks if i < shared_rows else 0) for i, n in enumerate(need))
    num_blocks = num_blocks or least
    assert num_blocks >= least
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    prefix, pos = perm[:shared_blocks], shared_blocks
    tables = torch.zeros(len(ctx), max(need), dtype=torch.int32)
    for i, n in enumerate(need):
        own = n - (shared_blocks if i < shared_rows else 0)
        row = (prefix if i < shared_rows else []) + perm[pos : pos + own]
        pos += own
        tables[i, :n] = torch.tensor(row, dtype=torch.int32)
    return tables, num_blocks


@pytest.mark.gpu
def test_load_workload_paged_prefill_matches_oracle(device):
    """One paged prefill launch over the whole batch: rows 0-49 query their last 1024 tokens over the
    shared 1024-token prefix, rows 50-99 their whole 2048-token prompt."""
    hq, hkv = 16, 8
    lens = [PROMPT] * N
    cached = [SHARED] * (N // 2) + [0] * (N // 2)
    tables, num_blocks = _shared_tables(lens, N // 2, SHARED // BS, seed=4)
    gen = torch.Generator(device=device).manual_seed(4)

    def rand(shape):
        return torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)

    q, k, v = rand((N * PROMPT, hq, 128)), rand((N * PROMPT, hkv, 128)), rand((N * PROMPT, hkv, 128))
    # the sharing rows' prefix tokens are one prompt's (they hit the same cached blocks)
    for i in range(1, N // 2):
        k[i * PROMPT : i * PROMPT + SHARED] = k[:SHARED]
        v[i * PROMPT : i * PROMPT + SHARED] = v[:SHARED]
    kc = torch.full((num_blocks, BS, hkv, 128), float("nan"), dtype=torch.bfloat16, device=device)
    vc = torch.full_like(kc, float("nan"))
    pos = torch.arange(PROMPT)
    slots = (tables[:, pos // BS].long() * BS + (pos % BS)).reshape(-1).to(device)
    _C.kv_cache_write(k, v, kc, vc, slots)
    sel = torch.cat([torch.arange(i * PROMPT + c, (i + 1) * PROMPT) for i, c in enumerate(cached)]).to(device)
    qs = q[sel].contiguous()
    q_lens = [n - c for n, c in zip(lens, cached)]
    cu_q = W.cu_seqlens(q_lens)
    out = torch.empty_like(qs)
    _C.paged_prefill(out, qs, kc, vc, tables.to(device), torch.tensor(cu_q, dtype=torch.int32, device=device),
                     torch.tensor(lens, dtype=torch.int32, device=device), max(q_lens), SCALE)
    dense = torch.empty_like(q)
    _C.varlen_prefill(dense, q, k, v, torch.tensor(W.cu_seqlens(lens), dtype=torch.int32, device=device), PROMPT,
                      SCALE)
    torch.cuda.synchronize()
    # every row of the batch: paged over the shared pages == dense over the whole prompt
    all_err = (out.float() - dense[sel].float()).abs().max().item()
    # 8 sequences against the oracle: 4 sharing the prefix, 4 not
    rows = [0, 1, 25, 49, 50, 51, 75, 99]
    errs = []
    kc_cpu, vc_cpu = kc.cpu(), vc.cpu()
    for i in rows:
        a, b = cu_q[i], cu_q[i + 1]
        ref = paged_prefill_ref(qs[a:b].cpu(), kc_cpu, vc_cpu, tables[i : i + 1], [0, b - a], [lens[i]], SCALE)
        errs.append((out[a:b].float().cpu() - ref).abs().max().item())
    print(f"[load prefill] {len(qs)} query rows; oracle max-abs per row {['%.3g' % e for e in errs]}; "
          f"paged vs dense over all rows {all_err:.3g}", flush=True)
    assert max(errs) <= TOL
    assert all_err <= TOL


def _decode_case(device):
    rng = random.Random(11)
    ctx = [rng.randint(2048, 4096) for _ in range(N)]
    # a pool as large as private pages would need (the seeded workload draws from it), shared rows
    # taking fewer of its blocks
    num_blocks = sum(-(-c // BS) for c in ctx) + 8
    tables, _ = _shared_tables(ctx, N // 2, SHARED // BS, seed=11, num_blocks=num_blocks)
    return ctx, tables, num_blocks


@pytest.mark.gpu
def test_load_workload_decode_matches_oracle(device):
    ctx, tables, num_blocks = _decode_case(device)
    work = W.make_decode(N, 0, 0, num_blocks, seed=11, device=device, context_lens=ctx)
    work.block_tables = tables.to(device)
    max_ctx = 4096
    ws = _C.alloc_paged_decode_workspace(N, 16, 8, max_ctx, device)
    out = torch.empty_like(work.q)
    _C.paged_decode(out, work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens, SCALE,
                    max_ctx, ws)
    torch.cuda.synchronize()
    ref = paged_decode_ref(work.q, work.key_cache[0], work.value_cache[0], tables, work.context_lens, SCALE)
    err = (out.float().cpu() - ref).abs().max().item()
    print(f"[load decode] 100 x U[2048, 4096] (sum {sum(ctx)} tokens), shared prefix pages: max-abs {err:.3g}",
          flush=True)
    assert err <= TOL


@pytest.mark.gpu
def test_load_workload_fused_decode_step_matches_oracle(device):
    ctx, tables, num_blocks = _decode_case(device)
    case = Case(device, N, 0, 0, num_blocks, seed=11, context_lens=ctx)
    case.work.block_tables = tables.to(device)
    bt = tables
    pos = [c - 1 for c in ctx]
    case.positions = torch.tensor(pos, dtype=torch.int64, device=device)
    case.slots = torch.tensor([int(bt[i, p // BS]) * BS + p % BS for i, p in enumerate(pos)], dtype=torch.int64,
                              device=device)
    out, kc, vc = case.fused(4096)
    chain, kc2, vc2 = case.unfused(4096)
    torch.cuda.synchronize()
    ref = case.oracle()
    err = (out.float().cpu() - ref).abs().max().item()
    print(f"[load fused decode] max-abs vs oracle {err:.3g}", flush=True)
    assert err <= TOL
    assert torch.equal(out, chain) and torch.equal(kc, kc2) and torch.equal(vc, vc2)
