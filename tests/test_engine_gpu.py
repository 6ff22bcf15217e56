"""End-to-end generation through the HIP path: greedy parity, graph == eager, prefix cache == no cache."""
from __future__ import annotations

import random
import sys
from dataclasses import replace
from pathlib import Path

import pytest
import torch

from nano_vllm_ascend_amd import LLM
from nano_vllm_ascend_amd.config import QWEN3_0_6B
from oracle.qwen3_ref import Qwen3Ref

sys.path.insert(0, str(Path(__file__).resolve().parent))
import greedy_bar  # noqa: E402

SMALL = replace(QWEN3_0_6B, num_hidden_layers=2)  # the 0.6B layer shape and vocabulary, 2 layers


def prompts_for(lens, seed=0):
    rng = random.Random(seed)
    return [[rng.randint(0, 10000) for _ in range(n)] for n in lens]


def make_llm(graph=True, prefix=False, layers=SMALL, num_blocks=96, max_num_seqs=8, seed=1, max_model_len=1024):
    return LLM(layers, max_model_len=max_model_len, num_blocks=num_blocks, max_num_seqs=max_num_seqs,
               enable_decode_graph=graph, enable_prefix_cache=prefix, seed=seed, retain_logits=True)


# Per-step logits of the 2-layer model against the oracle's (both bf16 values; one bf16 step of a
# logit near 3 is 0.0156): bf16 kernels whose fp32 summation order differs from the oracle's move a
# logit by a few hundredths at most (measured worst per step: 0.031 before the bf16 rounding).
LOGIT_TOL = 0.08
# Two product paths (fused and unfused decode projections) compared with each other: a token may
# differ only where the top two bf16 logits are within three bf16 steps (0.047 near 3).
TIE_TOL = 0.05


@pytest.mark.gpu
def test_greedy_tokens_match_oracle_for_32_decode_steps(device):
    """2-layer model, 4 prompts of 5-200 tokens, the prefill token plus 32 greedy decode steps, against
    the oracle under the bar derived from the oracle's own disagreement (tests/greedy_bar.py)."""
    llm = make_llm()
    llm.runner.tokenizer.eos_token_id = -1
    prompts = prompts_for([37, 128, 200, 5], seed=3)
    ids = [llm.submit(p, max_new_tokens=33) for p in prompts]  # the prefill token + 32 decode steps
    step_logits = _run_collecting_logits(llm, 33)
    tokens = [llm.scheduler.finished[i].generated_token_ids for i in ids]
    state = {k: v for k, v in llm.runner.model.state_dict().items()}
    variants = greedy_bar.legal_variants(state, SMALL, prompts, tokens, "cpu")
    greedy_bar.check(torch.stack(step_logits, dim=1), tokens, variants, "2-layer greedy")


def _run_collecting_logits(llm, steps):
    """Step the engine to the end; the logits of its first `steps` forwards (the prefill, then decode)."""
    step_logits = []
    while llm.has_unfinished():
        llm.step()
        if len(step_logits) < steps:
            step_logits.append(llm.runner.last_logits.float().cpu())
    return step_logits


# Other Qwen3 head layouts, 2 layers each: 40 query / 8 kv heads (Qwen3-14B's ratio 5) on the
# 0.6B hidden size, which takes the fused decode path; 32 / 4 heads (ratio 8) on Qwen3-4B's hidden
# and MLP sizes, which takes the unfused one.  Both run attention as several launches per layer.
WIDE_GQA = {
    "gqa5_fused": replace(QWEN3_0_6B, num_hidden_layers=2, num_attention_heads=40, num_key_value_heads=8),
    "gqa8_unfused": replace(QWEN3_0_6B, num_hidden_layers=2, num_attention_heads=32, num_key_value_heads=4,
                            hidden_size=2560, intermediate_size=9728),
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(WIDE_GQA))
def test_other_gqa_ratios_match_oracle(device, name):
    cfg = WIDE_GQA[name]
    llm = make_llm(layers=cfg)
    llm.runner.tokenizer.eos_token_id = -1
    fused = llm.runner.model.decode_fusable(2)
    assert fused == (name == "gqa5_fused")
    prompts = prompts_for([37, 150], seed=5)
    ids = [llm.submit(p, max_new_tokens=17) for p in prompts]
    step_logits = _run_collecting_logits(llm, 17)
    tokens = [llm.scheduler.finished[i].generated_token_ids for i in ids]
    state = {k: v for k, v in llm.runner.model.state_dict().items()}
    variants = greedy_bar.legal_variants(state, cfg, prompts, tokens, "cpu")
    greedy_bar.check(torch.stack(step_logits, dim=1), tokens, variants, name)


@pytest.mark.gpu
def test_decode_logits_match_oracle_each_step(device):
    llm = make_llm()
    llm.runner.tokenizer.eos_token_id = -1
    prompt = prompts_for([150], seed=11)[0]
    llm.submit(prompt, max_new_tokens=33)
    ref = Qwen3Ref({k: v for k, v in llm.runner.model.state_dict().items()}, SMALL, round_bf16=True,
                   max_positions=512)
    ref_logits = ref.forward(prompt)
    worst, steps = 0.0, 0
    seq = None
    while llm.has_unfinished():
        llm.step()
        seq = seq or next(iter(llm.scheduler.seqs.values()))
        if seq.finish_reason is not None:
            break
        got = llm.runner.last_logits[0].float().cpu()
        worst = max(worst, (got - ref_logits).abs().max().item())
        steps += 1
        ref_logits = ref.forward([seq.next_token_id])  # the token just sampled feeds the next step
    print(f"decode logits: {steps} steps, worst max-abs {worst:.4f}")
    assert steps == 33 and worst <= LOGIT_TOL


@pytest.mark.gpu
def test_graph_replay_equals_eager_and_counts(device):
    prompts = prompts_for([20, 129, 64, 300], seed=5)
    budgets = [3, 9, 6, 12]  # the decode batch shrinks 4 -> 3 -> 2 -> 1 (3 is not a captured size)

    def run(graph):
        llm = make_llm(graph=graph)
        llm.runner.tokenizer.eos_token_id = -1
        ids = [llm.submit(p, max_new_tokens=n) for p, n in zip(prompts, budgets)]
        res = {}
        while llm.has_unfinished():
            for o in llm.step():
                res[o["request_id"]] = o["token_ids"]
        return [res[i] for i in ids], llm.runner.decode_graph_stats()

    got, stats = run(True)
    ref, _ = run(False)
    assert got == ref
    assert [len(t) for t in got] == budgets
    assert stats["captures"] == 3 and stats["capture_failures"] == 0
    assert stats["fallbacks"] > 0 and stats["replays"] == stats["updates"] > 0


@pytest.mark.gpu
def test_prefix_cache_hit_equals_no_cache(device):
    shared = prompts_for([256], seed=7)[0]  # two full 128-token blocks
    tails = prompts_for([40, 97, 3], seed=8)
    cached_llm = make_llm(prefix=True)
    cached_llm.runner.tokenizer.eos_token_id = -1
    cached_llm.generate([shared + [1, 2, 3]], max_new_tokens=2)  # fills the prefix cache
    hit = cached_llm.generate([shared + t for t in tails], max_new_tokens=16)
    seqs = cached_llm.scheduler.finished
    assert all(s.cached_prefix_len == 256 for s in seqs.values())
    plain = make_llm(prefix=False)
    plain.runner.tokenizer.eos_token_id = -1
    miss = plain.generate([shared + t for t in tails], max_new_tokens=16)
    assert [o["token_ids"] for o in hit] == [o["token_ids"] for o in miss]


@pytest.mark.gpu
def test_full_depth_greedy_tokens_against_oracle(device):
    """The 32 x 256 / 2048 workload's model and prompts: Qwen3-0.6B shape (28 layers), seeded
    N(0, 0.02) weights (seed 0), the 32 prompts of 256 ids in [0, 10000] (seed 0).  The product
    runs free: the prefill token plus 32 greedy decode steps through the batch-32 decode graph,
    each step fed its own previous token.  The oracle (bf16 mode, on the GPU) is evaluated four
    legal ways on the product's token stream, and the product must stay within the disagreement
    of those evaluations with each other (tests/greedy_bar.py)."""
    from nano_vllm_ascend_amd.bench_e2e import make_dataset

    steps = 33
    prompts = make_dataset(32, 256, QWEN3_0_6B.vocab_size, seed=0)
    llm = LLM(QWEN3_0_6B, max_model_len=2304, num_blocks=32 * 3 + 8, max_num_seqs=32, seed=0, retain_logits=True)
    llm.runner.tokenizer.eos_token_id = -1
    ids = [llm.submit(p, max_new_tokens=steps) for p in prompts]
    step_logits = _run_collecting_logits(llm, steps)
    tokens = [llm.scheduler.finished[i].generated_token_ids for i in ids]
    stats = llm.runner.decode_graph_stats()
    assert stats["captures"] == 1 and stats["replays"] >= steps - 1 and stats["fallbacks"] == 0
    assert all(len(t) == steps for t in tokens)
    state = {k: v for k, v in llm.runner.model.state_dict().items()}
    del llm
    torch.cuda.empty_cache()
    variants = greedy_bar.legal_variants(state, QWEN3_0_6B, prompts, tokens, device)
    greedy_bar.check(torch.stack(step_logits, dim=1), tokens, variants, "full-depth greedy")


@pytest.mark.gpu
@pytest.mark.parametrize("n_prompts", [4, 100])
def test_fused_decode_path_matches_unfused_chain(device, n_prompts):
    """Decode batches <= 128 rows fold every RMSNorm and residual add into the projections (at
    100 rows: two 64-row slabs per projection); the logits must match the unfused chain
    (library GEMMs + add_rms_norm) of the same model to rounding, and tokens may differ only at
    near-ties."""
    kw = dict(graph=False) if n_prompts <= 8 else dict(graph=False, max_num_seqs=n_prompts, num_blocks=n_prompts * 3)
    fused, plain = make_llm(**kw), make_llm(**kw)
    plain.runner.model.decode_fusable = lambda rows: False
    lens = [37, 128, 200, 5] if n_prompts == 4 else [random.Random(i).randint(5, 250) for i in range(n_prompts)]
    prompts = prompts_for(lens, seed=3)
    for llm in (fused, plain):
        llm.runner.tokenizer.eos_token_id = -1
        for p in prompts:
            llm.submit(p, max_new_tokens=17)
    # Rows are independent (attention per sequence, GEMM rows), so a row whose token differs at a
    # near-tie leaves the comparison and the others go on.
    worst, steps, live, dropped = 0.0, 0, set(range(n_prompts)), 0
    while fused.has_unfinished():
        fused.step()
        plain.step()
        if not fused.has_unfinished():
            break  # the last step only commits final tokens
        la, lb = fused.runner.last_logits.float(), plain.runner.last_logits.float()
        assert la.shape == lb.shape == (n_prompts, la.shape[1])
        rows = sorted(live)
        if steps > 0 and rows:  # the first step is the (shared, unfused) prefill
            worst = max(worst, (la[rows] - lb[rows]).abs().max().item())
        steps += 1
        ta = [s.next_token_id for s in fused.scheduler.seqs.values()]
        tb = [s.next_token_id for s in plain.scheduler.seqs.values()]
        for row in rows:
            if ta[row] != tb[row]:
                assert (lb[row, tb[row]] - lb[row, ta[row]]).item() < TIE_TOL
                live.discard(row)
                dropped += 1
    print(f"fused vs unfused decode at {n_prompts} rows: {steps} steps, worst logit diff {worst:.4f}, "
          f"{dropped} rows left at near-ties")
    assert fused.runner.model._gemm_workspace is not None and plain.runner.model._gemm_workspace is None
    assert steps >= 16 and worst <= 0.05 and len(live) >= n_prompts // 2


@pytest.mark.gpu
def test_overlapped_decode_equals_synchronous_loop(device):
    """Launching step N+1 before step N's tokens reach the host changes nothing observable: the
    same tokens (including a request that stops on EOS mid-run, which discards the step launched
    ahead), and the per-step logits the runner exposes are those of the step just taken."""
    prompts = prompts_for([20, 129, 64, 300], seed=5)
    budgets = [7, 19, 13, 25]

    def run(overlap, eos=-1):
        llm = make_llm(graph=True)
        llm.runner.enable_overlap = overlap
        llm.runner.tokenizer.eos_token_id = eos
        ids = [llm.submit(p, max_new_tokens=n) for p, n in zip(prompts, budgets)]
        res, logits = {}, []
        while llm.has_unfinished():
            for o in llm.step():
                res[o["request_id"]] = o["token_ids"]
            if llm.runner.last_logits is not None:
                logits.append(llm.runner.last_logits.float().cpu().clone())
        return [res[i] for i in ids], logits, dict(llm.runner.overlap_stats)

    sync_tokens, sync_logits, sync_stats = run(False)
    tokens, logits, stats = run(True)
    assert tokens == sync_tokens
    assert len(logits) == len(sync_logits) and all(torch.equal(a, b) for a, b in zip(logits, sync_logits))
    assert sync_stats["launched"] == 0 and stats["launched"] > 0 and stats["used"] > 0
    # an EOS that the host only learns after the next step was launched: the launch is discarded
    eos = sync_tokens[3][20]  # late in the longest request, when a step has been launched ahead
    eos_sync, _, _ = run(False, eos=eos)
    eos_tokens, _, eos_stats = run(True, eos=eos)
    assert eos_tokens == eos_sync and eos_stats["discarded"] > 0
