"""End-to-end throughput of continuous-batching generation (workload of examples/bench_compare.py:191-325).

N requests of `input_len` random token ids (random.Random(seed), ids uniform
in [0, min(10000, vocab-1)]) submitted as token ids, greedy decoding with EOS
ignored for exactly `output_len` tokens each, one untimed warm-up run of the
same workload, then `output_tok_s = total generated tokens / elapsed` over one
timed run (prefill included).  The model is the Qwen3-0.6B shape with seeded
random weights.

    python -m nano_vllm_ascend_amd.bench_e2e --prompts 32 --input 256 --output 2048

The load workload -- 100 requests x 2048 / 2048 tokens, half of them sharing one
seeded 1024-token prefix, prefix cache on (the reference's own run of 100 x
2048 / 2048 is bench_outputs/nano_100_2048_2048.json) -- is

    python -m nano_vllm_ascend_amd.bench_e2e --prompts 100 --input 2048 --output 2048 \
        --shared-prefix 1024 --shared-fraction 0.5 --prefix-cache --graph-sizes 1,2,4,8,16,32,64,100

With the prefix cache on, the warm-up uses a different seed and a short output,
the cache is cleared, and then one seed request carrying the shared prefix is run
(its prefill caches the prefix's full blocks), so in the timed run exactly the
requests that share the prefix hit it.  The prefix lookup happens at submit time
and blocks are cached only after their prefill (nv/model_runner.py:146-167,
232-238), so without the seed request a run that submits everything before any
prefill could not hit at all.  The result reports the hits.  ``--graph-sizes``
sets the captured decode batch sizes (the load workload captures its batch of 100).
"""
from __future__ import annotations

import argparse
import json
import random
import time

import torch

from .config import QWEN3_0_6B
from .engine import LLM


def make_dataset(num_prompts: int, input_len: int, vocab_size: int, seed: int, token_id_high: int = 10000,
                 shared_prefix: int = 0, shared_fraction: float = 0.0):
    """Random prompts; the first round(shared_fraction * N) of them start with one common
    `shared_prefix`-token prefix (seeded too)."""
    rng = random.Random(seed)
    high = min(token_id_high, vocab_size - 1)
    prompts = [[rng.randint(0, high) for _ in range(input_len)] for _ in range(num_prompts)]
    if shared_prefix > 0 and shared_fraction > 0:
        prefix = [rng.randint(0, high) for _ in range(min(shared_prefix, input_len))]
        for p in prompts[: round(shared_fraction * num_prompts)]:
            p[: len(prefix)] = prefix
    return prompts


def generate_from_token_ids(llm: LLM, prompts: list[list[int]], output_len: int, sampling_params=None):
    """Run prompts given as token ids to completion (``LLM.generate``); generated ids per request."""
    return [o["token_ids"] for o in llm.generate(prompts, max_new_tokens=output_len, sampling_params=sampling_params)]


def run_e2e(num_prompts: int = 32, input_len: int = 256, output_len: int = 2048, seed: int = 0, device=None,
            max_model_len: int = 4096, block_size: int = 128, warmup: int = 1, num_blocks: int | None = None,
            enable_decode_graph: bool = True, llm: LLM | None = None, shared_prefix: int = 0,
            shared_fraction: float = 0.0, enable_prefix_cache: bool = False,
            graph_sizes: list[int] | None = None, config=None) -> dict:
    cfg = config or QWEN3_0_6B
    need = num_prompts * -(-(input_len + output_len) // block_size)
    if llm is None:
        llm = LLM(cfg, max_model_len=max_model_len, block_size=block_size, num_blocks=num_blocks or need + 64,
                  max_num_seqs=num_prompts, enable_decode_graph=enable_decode_graph, seed=seed,
                  enable_prefix_cache=enable_prefix_cache, decode_graph_batch_sizes=graph_sizes)
    llm.runner.tokenizer.eos_token_id = -1  # ignore EOS, as the reference benchmark does
    prompts = make_dataset(num_prompts, input_len, cfg.vocab_size, seed, shared_prefix=shared_prefix,
                           shared_fraction=shared_fraction)
    for w in range(warmup):
        if enable_prefix_cache:  # other prompts and a short output: graphs captured, nothing cached that hits
            warm = make_dataset(num_prompts, input_len, cfg.vocab_size, seed + 1 + w, shared_prefix=shared_prefix,
                                shared_fraction=shared_fraction)
            generate_from_token_ids(llm, warm, min(output_len, 16))
        else:
            generate_from_token_ids(llm, prompts, output_len)
        torch.cuda.synchronize()
    seeded = 0
    if enable_prefix_cache:
        llm.clear_prefix_cache()
        if shared_prefix and shared_fraction:
            # one seed request carrying the shared prefix caches its full blocks
            n_shared = round(shared_fraction * num_prompts)
            seed_prompt = prompts[0][: shared_prefix] + [prompts[n_shared % num_prompts][0]]
            generate_from_token_ids(llm, [seed_prompt], 1)
            seeded = shared_prefix // block_size
        torch.cuda.synchronize()
    graph0 = dict(llm.runner.decode_graph_stats())
    prefill0 = dict(llm.runner.prefill_stats)
    t0 = time.perf_counter()
    outs = generate_from_token_ids(llm, prompts, output_len)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    generated = sum(len(o) for o in outs)
    workload = f"{num_prompts}x{input_len}/{output_len} greedy ignore_eos"
    if shared_prefix and shared_fraction:
        workload += f", {shared_fraction:g} of requests share a {shared_prefix}-token prefix"
    if enable_prefix_cache:
        workload += ", prefix cache on" + (", warmed by one seed request carrying the prefix" if seeded else "")
    seqs = list(llm.scheduler.finished.values())
    hits = [s for s in seqs if s.cached_prefix_len > 0]
    graph = {k: v - graph0.get(k, 0) for k, v in llm.runner.decode_graph_stats().items()}
    prefill = {k: v - prefill0.get(k, 0) for k, v in llm.runner.prefill_stats.items()}
    return {
        "workload": workload,
        "output_tok_s": round(generated / elapsed, 2),
        "total_tok_s": round((generated + num_prompts * input_len) / elapsed, 2),
        "elapsed_s": round(elapsed, 3),
        "generated_tokens": generated,
        "decode_graph": llm.runner.decode_graph_stats(),  # the whole run, warm-up included
        "decode_graph_timed": graph,
        "decode_graph_batch_sizes": sorted(llm.runner.decode_graph_runner.batch_sizes)
        if llm.runner.decode_graph_runner is not None else [],
        "overlapped_steps": dict(llm.runner.overlap_stats),
        "prefix_cache": {"requests_with_hits": len(hits), "hit_blocks": sum(len(s.cached_block_ids) for s in hits),
                         "hit_tokens": sum(s.cached_prefix_len for s in hits), "prefill": prefill}
        if enable_prefix_cache else None,
        "model": "Qwen3-0.6B shape, seeded N(0, 0.02) weights, bf16",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--prompts", type=int, default=32)
    ap.add_argument("--input", type=int, default=256)
    ap.add_argument("--output", type=int, default=2048)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--shared-prefix", type=int, default=0, help="tokens of the common prefix")
    ap.add_argument("--shared-fraction", type=float, default=0.0, help="fraction of requests that share it")
    ap.add_argument("--prefix-cache", action="store_true")
    ap.add_argument("--max-model-len", type=int, default=4096)
    ap.add_argument("--graph-sizes", type=str, default=None,
                    help="comma-separated captured decode batch sizes (default: 1,2,4,8,16,32)")
    args = ap.parse_args()
    sizes = [int(x) for x in args.graph_sizes.split(",")] if args.graph_sizes else None
    print(json.dumps(run_e2e(args.prompts, args.input, args.output, args.seed, warmup=args.warmup,
                             enable_decode_graph=not args.no_graph, shared_prefix=args.shared_prefix,
                             shared_fraction=args.shared_fraction, enable_prefix_cache=args.prefix_cache,
                             max_model_len=args.max_model_len, graph_sizes=sizes)))


if __name__ == "__main__":
    main()
