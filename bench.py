"""Benchmark of the MI355X continuous-batching attention path.

One JSON line on stdout.  `value` is paged decode attention throughput in
GB/s of algorithmic HBM traffic (K/V read once per kv head and context token,
q read, out written, block tables and context lengths read), over a decode
step of 32 sequences with context lengths uniform in [256, 2304] run through
all 28 layers' KV caches of a Qwen3-0.6B-shaped model (16 q / 8 kv heads,
head_dim 128, block_size 128, bf16): one "step" = 28 launches, one per layer,
each reading its own layer's pages so the 256 MB Infinity Cache cannot serve
them.  Inputs are resident in HBM before the timed region.

Also reported: the roofline of the decode kernel (average launch duration from
HIP events on the launch stream), the fp32 CPU oracle on the host cores as the
CPU baseline, the same decode step with the per-head q/k norm, RoPE and KV store fused into
the attention launch (against the two-launch chain), the same kernel at larger decode shapes (up
to the load workload's 100 sequences x U[2048, 4096]), the ragged causal prefill of 32 prompts of U[64, 2048] tokens
(TFLOP/s against the dense bf16 MFMA peak) with its paged KV store (GB/s), and
(unless --no-e2e) the end-to-end output tok/s of the 32 x 256-in / 2048-out
greedy workload and of the 100 x 2048 / 2048 load workload (half the requests share
a 1024-token prefix, prefix cache on, batch-100 decode graph; unless --no-load),
each next to the reference's published 910B3 figure, with truncated runs of the
fp32 CPU oracle model on the same weights beside them.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
REFERENCE_E2E_TOK_S = 1296.05  # nano_vllm_ascend on Ascend 910B3, 32 x 256/2048, bench_outputs/nano_32x256_2048.json
REFERENCE_LOAD_TOK_S = 1410.23  # the same on 100 x 2048/2048 (batch-100 graph), bench_outputs/nano_100_2048_2048.json
NUM_LAYERS = 28


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end generation leg")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill leg")
    ap.add_argument("--e2e-prompts", type=int, default=32)
    ap.add_argument("--e2e-input", type=int, default=256)
    ap.add_argument("--e2e-output", type=int, default=2048)
    ap.add_argument("--no-load", action="store_true",
                    help="skip the 100 x 2048/2048 shared-prefix workload (prefix cache on, batch-100 graph)")
    ap.add_argument("--load-output", type=int, default=2048)
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="only run 5 device copies of MB megabytes (calibrates HBM byte counters), then exit")
    return ap.parse_args()


def copy_probe(mb: int) -> None:
    """A plain device-to-device copy of known size: MB*2^20 bytes read and written per launch."""
    import torch

    n = mb * (1 << 20)
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "launches": 5}))


def kernel_source_sha(name: str) -> str:
    import hashlib

    return hashlib.sha256((ROOT / "nano_vllm_ascend_amd" / "csrc" / name).read_bytes()).hexdigest()[:16]


def load_traffic(workload: str) -> tuple[float | None, str]:
    """HBM bytes per launch from rocprofv3 PMC counters (FETCH_SIZE, WRITE_SIZE runs; committed under
    profiles/traffic.json with the hash of the kernel source they were measured on) and where the
    figure comes from.  A figure measured on another version of the source is stale: None."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None, "no profiles/traffic.json"
    try:
        entry = json.loads(path.read_text()).get(workload)
    except ValueError:
        return None, "profiles/traffic.json unreadable"
    if entry is None:
        return None, f"no entry for {workload} in profiles/traffic.json"
    src = entry.get("kernel_source", "paged_decode.hip")
    if entry.get("kernel_source_sha256") != kernel_source_sha(src):
        return None, f"stale: profiles/traffic.json was measured on another version of csrc/{src}"
    return float(entry["bytes_per_launch"]), (f"rocprofv3 PMC (FETCH_SIZE x{entry['fetch_scale']:g}, WRITE_SIZE "
                                              f"x{entry['write_scale']:g}), {entry['source']}, csrc/{src} "
                                              f"sha256 {entry['kernel_source_sha256']}")


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def decode_leg(args, device):
    import torch

    from nano_vllm_ascend_amd import _C
    from nano_vllm_ascend_amd import workloads as W

    work = W.decode_step(device, seed=args.seed, num_layers=NUM_LAYERS)
    b = len(work.context_lens_list)
    max_ctx = max(work.context_lens_list)
    scale = W.HEAD_DIM ** -0.5
    ws = _C.alloc_paged_decode_workspace(b, W.NUM_HEADS, W.NUM_KV_HEADS, max_ctx, device)
    out = torch.empty_like(work.q)
    bytes_per_launch = (
        sum(work.context_lens_list) * W.NUM_KV_HEADS * W.HEAD_DIM * 2 * 2
        + 2 * b * W.NUM_HEADS * W.HEAD_DIM * 2
        + b * work.block_tables.shape[1] * 4
        + b * 4
    )
    layers = [(work.key_cache[l], work.value_cache[l]) for l in range(NUM_LAYERS)]
    stream = torch.cuda.current_stream()

    def step():
        for kc, vc in layers:
            _C.paged_decode(out, work.q, kc, vc, work.block_tables, work.context_lens, scale, max_ctx, ws)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # HIP events on the launch stream bracket the timed region; back-to-back launches of the
    # same kernel, so region time / launches is the kernel's average launch duration
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    start.record(stream)
    marks[0].record(stream)
    for i in range(args.steps):
        step()
        marks[i + 1].record(stream)
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    step_ms = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps))
    launches = args.steps * NUM_LAYERS
    avg_launch_s = total_ms / 1e3 / launches
    value = bytes_per_launch * launches / (total_ms / 1e3) / 1e9
    achieved = bytes_per_launch / avg_launch_s / 1e9
    return {
        "value": value,
        "ms_per_step": total_ms / args.steps,
        "bytes_per_launch": bytes_per_launch,
        "avg_launch_us": avg_launch_s * 1e6,
        "median_launch_us": step_ms[len(step_ms) // 2] * 1e3 / NUM_LAYERS,
        "achieved": achieved,
        "work": work,
        "max_ctx": max_ctx,
    }


def fused_step_leg(args, work, device) -> dict:
    """The decode step of the same 32 sequences as a model layer runs it: per-head q/k RMSNorm
    (eps 1e-6, weights N(1, 0.02)), RoPE (theta 1e6), the KV store of the new tokens through
    slot_mapping, then paged attention -- as two launches (qk_norm_rope with the store, then
    paged_decode) and as the one fused launch (nvamd_paged_decode_fused), over the 28 layers'
    pools.  HIP events around `steps` eager passes; microseconds per layer."""
    import torch

    from nano_vllm_ascend_amd import _C
    from nano_vllm_ascend_amd import workloads as W
    from nano_vllm_ascend_amd.layers import RotaryEmbedding

    inp = W.fused_step_inputs(work, args.seed, device)
    table = RotaryEmbedding(W.HEAD_DIM, 40960, W.ROPE_THETA).cos_sin.to(device)
    b = inp.qkv.shape[0]
    hq, hkv, d = W.NUM_HEADS, W.NUM_KV_HEADS, W.HEAD_DIM
    max_ctx = max(work.context_lens_list)
    scale = d ** -0.5
    ws = _C.alloc_paged_decode_workspace(b, hq, hkv, max_ctx, device)
    out = torch.empty(b, hq, d, dtype=torch.bfloat16, device=device)
    raw = inp.qkv
    def views(qkv):
        return (qkv[:, : hq * d].view(b, hq, d), qkv[:, hq * d : (hq + hkv) * d].view(b, hkv, d),
                qkv[:, (hq + hkv) * d :].view(b, hkv, d))

    q, k, v = views(raw)
    q2, k2, v2 = views(raw.clone())  # the two-launch chain rewrites q and k in place
    layers = [(work.key_cache[l], work.value_cache[l]) for l in range(NUM_LAYERS)]

    def two_launches():
        for kc, vc in layers:
            _C.qk_norm_rope(q2, k2, inp.q_weight, inp.k_weight, inp.positions, table, W.RMS_EPS, v=v2, key_cache=kc,
                            value_cache=vc, slot_mapping=inp.slot_mapping)
            _C.paged_decode(out, q2, kc, vc, work.block_tables, work.context_lens, scale, max_ctx, ws)

    def fused():
        for kc, vc in layers:
            _C.paged_decode_fused(out, q, k, v, inp.q_weight, inp.k_weight, inp.positions, table, W.RMS_EPS, kc, vc,
                                  inp.slot_mapping, work.block_tables, work.context_lens, scale, max_ctx, ws)

    def us_per_layer(fn, reps=20):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * NUM_LAYERS)

    two = us_per_layer(two_launches)
    one = us_per_layer(fused)
    # algorithmic bytes of the step: the attention's (K/V, raw q read once, out written, table row, context
    # length), plus per sequence the raw new k and v read, the new k/v stored, position and slot, and the
    # fp32 cos/sin row; and the two norm weights once
    step_bytes = (sum(work.context_lens_list) * hkv * d * 2 * 2 + 2 * b * hq * d * 2 + b * work.block_tables.shape[1] * 4
                  + b * 4 + b * (2 * hkv * d * 2 + 2 * hkv * d * 2 + 16 + d * 4) + 2 * d * 2)
    return {"workload": "decode step, 32 seqs, context U[256, 2304]: q/k norm + RoPE + KV store + attention",
            "two_launches_us_per_layer": round(two, 3), "fused_us_per_layer": round(one, 3),
            "saved_us_per_layer": round(two - one, 3), "bytes": step_bytes,
            "fused_gbs": round(step_bytes / one / 1e3, 1), "fused_frac": round(step_bytes / one / 1e3 / HBM_PEAK_GBS, 4)}


def small_decode_leg(args, device) -> dict:
    """Single-layer decode shape of 4 sequences, context U[1, 512], 64-block pools: as 28 launches
    (one per layer, each its own pool, 0.9 GB in total) captured in one hipGraph, and as one eager
    launch, which is latency-bound.  Medians over 50 replays / launches after 5 warm-ups."""
    import torch

    from nano_vllm_ascend_amd import _C
    from nano_vllm_ascend_amd import workloads as W

    work = W.make_decode(4, 1, 512, 64, args.seed, device, num_layers=NUM_LAYERS)
    b = len(work.context_lens_list)
    max_ctx = 512
    scale = W.HEAD_DIM ** -0.5
    ws = _C.alloc_paged_decode_workspace(b, W.NUM_HEADS, W.NUM_KV_HEADS, max_ctx, device)
    out = torch.empty_like(work.q)
    nbytes = (sum(work.context_lens_list) * W.NUM_KV_HEADS * W.HEAD_DIM * 2 * 2 + 2 * b * W.NUM_HEADS * W.HEAD_DIM * 2
              + b * work.block_tables.shape[1] * 4 + b * 4)

    def launch(layer):
        _C.paged_decode(out, work.q, work.key_cache[layer], work.value_cache[layer], work.block_tables,
                        work.context_lens, scale, max_ctx, ws)

    for layer in range(NUM_LAYERS):  # eager warm-up outside the capture
        launch(layer)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for layer in range(NUM_LAYERS):
            launch(layer)

    def median_ms(fn, reps=50, warm=5):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        ev[0].record()
        for i in range(reps):
            fn()
            ev[i + 1].record()
        torch.cuda.synchronize()
        t = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))
        return t[len(t) // 2]

    graph_us = median_ms(graph.replay) * 1e3 / NUM_LAYERS
    single_us = median_ms(lambda: launch(0)) * 1e3
    return {
        "workload": "decode 4 seqs, context U[1, 512] (sum %d), 64-block pools" % sum(work.context_lens_list),
        "bytes_per_launch": nbytes,
        "graph_28_layers": {"us_per_launch": round(graph_us, 3), "gbs": round(nbytes / graph_us / 1e3, 1),
                            "frac": round(nbytes / graph_us / 1e3 / HBM_PEAK_GBS, 4)},
        "single_launch": {"us": round(single_us, 3), "gbs": round(nbytes / single_us / 1e3, 1),
                          "note": "latency-bound: one small launch"},
        "work": work,
    }


# Other decode shapes for the same kernel: the 32-sequence step at twice the batch, at the load
# workload's context range (2048 prompt tokens + up to 2048 generated) and at that workload's batch
# of 100; and one rank's share of the 32-sequence step under 8-way head parallelism (2 query heads,
# 1 kv head).  Each shape rotates over `layers` pools whose summed read set is far beyond the 256 MB
# Infinity Cache.  (batch, context lo, context hi, layers, query heads, kv heads)
SCALING_SHAPES = ((64, 256, 2304, 14, 16, 8), (32, 2048, 4096, 10, 16, 8), (100, 2048, 4096, 4, 16, 8),
                  (32, 256, 2304, 28, 2, 1))


def decode_scaling_leg(args, device) -> list[dict]:
    """GB/s of the decode kernel at other shapes (average over the launches of graph replays, HIP
    events on the launch stream): how much of the 32-sequence step's gap to the HBM peak is the
    launch's fixed ramp and merge tail, which larger launches amortise."""
    import torch

    from nano_vllm_ascend_amd import _C
    from nano_vllm_ascend_amd import workloads as W

    rows = []
    for batch, lo, hi, layers, hq, hkv in SCALING_SHAPES:
        work = W.make_decode(batch, lo, hi, batch * -(-hi // W.BLOCK_SIZE) + 8, args.seed, device, num_layers=layers,
                             num_heads=hq, num_kv_heads=hkv)
        max_ctx = max(work.context_lens_list)
        ws = _C.alloc_paged_decode_workspace(batch, hq, hkv, max_ctx, device)
        out = torch.empty_like(work.q)
        nbytes = (sum(work.context_lens_list) * hkv * W.HEAD_DIM * 2 * 2
                  + 2 * batch * hq * W.HEAD_DIM * 2 + batch * work.block_tables.shape[1] * 4 + batch * 4)
        scale = W.HEAD_DIM ** -0.5

        def step():
            for layer in range(layers):
                _C.paged_decode(out, work.q, work.key_cache[layer], work.value_cache[layer], work.block_tables,
                                work.context_lens, scale, max_ctx, ws)

        # replayed as one graph: the one-kv-head share's launches are shorter than a host-side
        # launch, which would otherwise set their pace
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        reps = max(5, args.steps * NUM_LAYERS // layers)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1e3 / (reps * layers)
        gbs = nbytes / us / 1e3
        rows.append({"workload": f"decode {batch} seqs, context U[{lo}, {hi}] (sum {sum(work.context_lens_list)}), "
                                 f"{hq} q / {hkv} kv heads, {layers} layer pools",
                     "bytes_per_launch": nbytes, "avg_launch_us": round(us, 3), "gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)})
        del work, ws, out
        torch.cuda.empty_cache()
    return rows


def prefill_leg(args, device) -> dict:
    """Ragged causal prefill: 32 prompts of U[64, 2048] tokens packed with cu_seqlens, 16 q / 8 kv
    heads, head_dim 128, bf16 N(0, 1); the K/V store into block_size-128 pages through a seeded
    slot mapping, then varlen attention.  Timed with HIP events over repeated launches."""
    import torch

    from nano_vllm_ascend_amd import _C
    from nano_vllm_ascend_amd import workloads as W

    lens = W.prefill_lengths(32, 64, 2048, seed=args.seed)
    t = sum(lens)
    gen = torch.Generator(device=device).manual_seed(args.seed)
    q = torch.randn(t, 16, 128, generator=gen, device=device).bfloat16()
    k = torch.randn(t, 8, 128, generator=gen, device=device).bfloat16()
    v = torch.randn(t, 8, 128, generator=gen, device=device).bfloat16()
    cu = torch.tensor(W.cu_seqlens(lens), dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    num_blocks = -(-t // 128) + 64
    kc = torch.zeros(num_blocks, 128, 8, 128, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    slots = torch.randperm(num_blocks * 128, generator=torch.Generator().manual_seed(args.seed))[:t].to(device)
    scale = 128 ** -0.5

    def timed(fn, reps, warmup=10):
        for _ in range(warmup):  # the first launches after other work run below full clocks
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / reps

    def rotating(fn, sets):
        # consecutive launches take different buffer sets (together well beyond the 256 MB
        # Infinity Cache), so each launch streams its bytes from HBM
        turn = [0]

        def call():
            fn(*sets[turn[0] % len(sets)])
            turn[0] += 1
        return call

    # ~20 launches (8 ms) of sustained MFMA work pass before the clocks settle
    us_attn = timed(lambda: _C.varlen_prefill(out, q, k, v, cu, max(lens), scale), 40, warmup=30)
    store_sets = [(k, v, kc, vc)] + [(k.clone(), v.clone(), torch.zeros_like(kc), torch.zeros_like(vc))
                                     for _ in range(2)]
    us_store = timed(rotating(lambda a, b, c, d: _C.kv_cache_write(a, b, c, d, slots), store_sets), 42)
    # the ceiling for these byte streams: a plain device copy of the same bytes, rotating likewise
    copy_sets = [(torch.empty(2 * k.numel(), dtype=k.dtype, device=device),
                  torch.cat([x[0].reshape(-1), x[1].reshape(-1)])) for x in store_sets]
    us_copy = timed(rotating(lambda d, s_: d.copy_(s_), copy_sets), 42)
    copy_gbs = 2 * (2 * k.numel() * 2) / us_copy / 1e3  # K and V bytes read + written per copy
    del copy_sets

    # per-head q/k RMSNorm + RoPE + KV store of the same tokens, on views into a fused
    # projection output [T, (16 + 2 * 8) * 128], in place
    from nano_vllm_ascend_amd.layers import RotaryEmbedding

    table = RotaryEmbedding(128, 40960, W.ROPE_THETA).cos_sin.to(device)
    qw = (1.0 + 0.02 * torch.randn(128, generator=gen, device=device)).bfloat16()
    kw = (1.0 + 0.02 * torch.randn(128, generator=gen, device=device)).bfloat16()
    pos = torch.tensor([p for n in lens for p in range(n)], dtype=torch.int64, device=device)
    norm_sets = []
    for _, _, c1, c2 in store_sets:
        qkv = torch.randn(t, 32 * 128, generator=gen, device=device).bfloat16()
        norm_sets.append((qkv[:, :2048].view(t, 16, 128), qkv[:, 2048:3072].view(t, 8, 128),
                          qkv[:, 3072:].view(t, 8, 128), c1, c2))
    us_norm = timed(rotating(lambda a, b, c, d, e: _C.qk_norm_rope(a, b, qw, kw, pos, table, W.RMS_EPS, v=c,
                                                                   key_cache=d, value_cache=e, slot_mapping=slots),
                             norm_sets), 42)
    norm_bytes = t * ((16 + 8) * 128 * 2 * 2 + 8 * 128 * 2 + 2 * 8 * 128 * 2 + 16)

    # paged (prefix-hit) route: 32 prompts of 1024 cached + 1024 new tokens through block tables
    pb, pq, pkv = 32, 1024, 2048
    pblocks = pb * (pkv // 128) + 16
    pkc = torch.randn(pblocks, 128, 8, 128, generator=gen, device=device).bfloat16()
    pvc = torch.randn(pblocks, 128, 8, 128, generator=gen, device=device).bfloat16()
    pbt = torch.randperm(pblocks, generator=torch.Generator().manual_seed(args.seed))[: pb * (pkv // 128)]
    pbt = pbt.view(pb, pkv // 128).to(torch.int32).to(device)
    pqq = torch.randn(pb * pq, 16, 128, generator=gen, device=device).bfloat16()
    pcu = torch.tensor([i * pq for i in range(pb + 1)], dtype=torch.int32, device=device)
    pkl = torch.full((pb,), pkv, dtype=torch.int32, device=device)
    pout = torch.empty_like(pqq)
    us_paged = timed(lambda: _C.paged_prefill(pout, pqq, pkc, pvc, pbt, pcu, pkl, pq, scale), 40, warmup=30)
    paged_flops = W.causal_attention_flops([pq] * pb, [pkv] * pb, 16)
    flops = W.causal_attention_flops(lens, lens, 16)
    store_bytes = t * 8 * 128 * 2 * 2 * 2 + t * 8  # K and V read + written, slot ids
    tflops = flops / us_attn / 1e6
    return {
        "workload": "ragged causal prefill, 32 prompts U[64, 2048] (seed %d), 16 q / 8 kv heads, d 128" % args.seed,
        "tokens": t,
        "attention": {"kernel": "prefill_kernel", "us": round(us_attn, 2), "flops": flops,
                      "tflops": round(tflops, 1), "bound": "mfma", "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                      "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)},
        "kv_store": {"kernel": "kv_cache_write_kernel", "us": round(us_store, 2), "bytes": store_bytes,
                     "gbs": round(store_bytes / us_store / 1e3, 1),
                     "frac": round(store_bytes / us_store / 1e3 / HBM_PEAK_GBS, 4),
                     "device_copy_gbs": round(copy_gbs, 1)},
        "qk_norm_rope": {"kernel": "qk_norm_rope_kernel (with the KV store)", "us": round(us_norm, 2),
                         "bytes": norm_bytes, "gbs": round(norm_bytes / us_norm / 1e3, 1),
                         "frac": round(norm_bytes / us_norm / 1e3 / HBM_PEAK_GBS, 4)},
        "paged_route": {"workload": "32 prompts x (1024 cached + 1024 new tokens), block_size 128",
                        "kernel": "prefill_kernel (paged)", "us": round(us_paged, 2), "flops": paged_flops,
                        "tflops": round(paged_flops / us_paged / 1e6, 1),
                        "frac": round(paged_flops / us_paged / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4)},
    }


def pack_leg(args, device) -> dict:
    """GPU packing of the batch metadata (slot_mapping, block_tables, context_lens, cu_seqlens,
    positions, input ids) by BlockManager: a ragged prefill of 32 prompts of U[64, 2048] tokens
    (token ids included) and a 32-row decode step, block_size 128.  Wall time per call with the
    host work, the one upload and the kernel, synchronised."""
    import random

    import torch

    from nano_vllm_ascend_amd import workloads as W
    from nano_vllm_ascend_amd.block_manager import BlockManager

    lens = W.prefill_lengths(32, 64, 2048, seed=args.seed)
    rng = random.Random(args.seed)
    tokens = [[rng.randint(0, 151935) for _ in range(n)] for n in lens]
    bm = BlockManager(num_blocks=1024, block_size=128, device=device)
    slots = list(range(32))

    def prefill():
        bm.prepare_prefill_metadata(slots, lens, [0] * 32, [[] for _ in slots], token_ids=tokens)
        torch.cuda.synchronize()

    def median_us(fn, reset=None, reps=20):
        times = []
        for i in range(reps + 3):
            t0 = time.perf_counter()
            fn()
            dt = time.perf_counter() - t0
            if reset is not None:
                reset()
            if i >= 3:
                times.append(dt)
        return sorted(times)[len(times) // 2] * 1e6

    def release():
        for s_ in slots:
            bm.free_slot(s_)

    us_prefill = median_us(prefill, reset=release)
    prefill()
    decode = lambda: (bm.prepare_decode_metadata(slots, list(lens), 1), torch.cuda.synchronize())
    us_decode = median_us(decode)
    return {"prefill_32_prompts_us": round(us_prefill, 1), "tokens": sum(lens),
            "decode_32_rows_us": round(us_decode, 1),
            "note": "wall time per call: host descriptors, one upload, pack kernel, synchronise"}


def cpu_baseline(work, seed: int, reps: int = 20):
    """fp32 oracle on the host cores: the 32-sequence decode step of one layer (layer 0 of the same
    batch), whole -- per-head q/k RMSNorm + RoPE, the new token's K/V written into its page
    (index_copy_ into the flattened cache, as PagedKVCache.write), paged decode attention -- and the
    attention alone; medians of `reps` runs after 3 warm-ups."""
    import torch

    from nano_vllm_ascend_amd import workloads as W
    from oracle.attention_ref import paged_decode_ref, qk_norm_rope_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    b = len(work.context_lens_list)
    bs = work.key_cache.shape[2]
    # Copy only the pages the batch reads (layer 0), renumbered densely, to host memory.
    bt = work.block_tables.cpu()
    need = [(c + bs - 1) // bs for c in work.context_lens_list]
    ids = torch.cat([bt[i, : need[i]] for i in range(b)]).long()
    kc = work.key_cache[0][ids.to(work.key_cache.device)].cpu()
    vc = work.value_cache[0][ids.to(work.value_cache.device)].cpu()
    tables = torch.zeros_like(bt)
    pos = 0
    for i in range(b):
        tables[i, : need[i]] = torch.arange(pos, pos + need[i], dtype=torch.int32)
        pos += need[i]
    inp = W.fused_step_inputs(work, seed, work.q.device)
    qkv = inp.qkv.cpu()
    q = qkv[:, : 16 * 128].view(b, 16, 128)
    k = qkv[:, 16 * 128: 24 * 128].view(b, 8, 128)
    v = qkv[:, 24 * 128:].view(b, 8, 128)
    qw, kw, positions = inp.q_weight.cpu(), inp.k_weight.cpu(), inp.positions.cpu()
    slots = torch.tensor([int(tables[i, p // bs]) * bs + p % bs for i, p in enumerate(positions.tolist())])
    ctx = work.context_lens.cpu()
    scale = 128 ** -0.5
    kflat, vflat = kc.view(-1, 8, 128), vc.view(-1, 8, 128)

    def step():
        qn, kn = qk_norm_rope_ref(q, k, qw, kw, positions, W.ROPE_THETA, W.RMS_EPS, 4096)
        kflat.index_copy_(0, slots, kn)
        vflat.index_copy_(0, slots, v)
        paged_decode_ref(qn, kc, vc, tables, ctx, scale)

    def attention():
        paged_decode_ref(work_q, kc, vc, tables, ctx, scale)

    work_q = work.q.cpu()

    def median(fn):
        for _ in range(3):
            fn()
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return sorted(times)[reps // 2]

    t_step, t_attn = median(step), median(attention)
    attn_bytes = sum(work.context_lens_list) * 8 * 128 * 2 * 2 + 2 * b * 16 * 128 * 2 + b * bt.shape[1] * 4 + b * 4
    step_bytes = attn_bytes + b * ((16 + 8) * 128 * 2 * 2 + 8 * 128 * 2 + 2 * 8 * 128 * 2 + 16)
    return {
        "value": round(step_bytes / t_step / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"fp32 torch-CPU oracle, the decode step of layer 0 of the same 32-sequence batch (q/k norm + "
                  f"RoPE + KV write + paged attention), median of {reps} after 3 warm-ups; GB/s of the step's "
                  f"algorithmic bytes",
        "step_ms": round(t_step * 1e3, 2),
        "attention_only": {"ms": round(t_attn * 1e3, 2), "gbs": round(attn_bytes / t_attn / 1e9, 3),
                           "note": "same bytes as the GPU value"},
        "cpu": cpu_model(),
    }


def cpu_baselines_other(small_work, seed: int, prefill_reps: int = 20) -> dict:
    """fp32 oracle on the host cores for the other decode shape, the ragged prefill and its KV write
    (the reference's index_copy_ into the flattened cache), each a median of 20 reps after 3 warm-ups."""
    import torch

    from nano_vllm_ascend_amd import workloads as W
    from oracle.attention_ref import paged_decode_ref, varlen_prefill_ref
    from oracle.block_manager_ref import BlockManagerRef

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    w = small_work
    q, kc, vc = w.q.cpu(), w.key_cache[0].cpu(), w.value_cache[0].cpu()
    bt, ctx = w.block_tables.cpu(), w.context_lens.cpu()
    scale = 128 ** -0.5
    for _ in range(3):
        paged_decode_ref(q, kc, vc, bt, ctx, scale)
    times = []
    for _ in range(20):
        t0 = time.perf_counter()
        paged_decode_ref(q, kc, vc, bt, ctx, scale)
        times.append(time.perf_counter() - t0)
    dec_s = sorted(times)[10]
    nbytes = sum(w.context_lens_list) * 8 * 128 * 4 + 2 * 4 * 16 * 128 * 2
    lens = W.prefill_lengths(32, 64, 2048, seed=seed)
    t = sum(lens)
    g = torch.Generator().manual_seed(seed)
    pq = torch.randn(t, 16, 128, generator=g).bfloat16()
    pk = torch.randn(t, 8, 128, generator=g).bfloat16()
    pv = torch.randn(t, 8, 128, generator=g).bfloat16()
    cu = torch.tensor(W.cu_seqlens(lens), dtype=torch.int32)

    def median(fn, reps):
        for _ in range(3):
            fn()
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return sorted(times)[reps // 2]

    pf_s = median(lambda: varlen_prefill_ref(pq, pk, pv, cu, scale), prefill_reps)
    # the prompts' K/V written into a 128-token-block cache through a seeded slot mapping, as
    # PagedKVCache.write does (nv/npu/paged_kv_cache.py:68-69: index_copy_ along the flattened slots)
    pool = W.seeded_block_tables(lens, 1024, 128, seed)
    kv_slots = torch.tensor([int(pool.block_tables[i, p // 128]) * 128 + p % 128 for i, n in enumerate(lens)
                             for p in range(n)], dtype=torch.int64)
    kcache = torch.zeros(1024 * 128, 8, 128, dtype=torch.bfloat16)
    vcache = torch.zeros_like(kcache)

    def kv_write():
        kcache.index_copy_(0, kv_slots, pk)
        vcache.index_copy_(0, kv_slots, pv)

    kv_s = median(kv_write, 20)
    kv_bytes = 2 * 2 * t * 8 * 128 * 2 + t * 8  # K and V read and written, and the slot mapping
    # reference-style packing: the per-token slot loop on the host
    bm = BlockManagerRef(1024, 128)
    slots = list(range(32))
    pack_times = []
    for i in range(8):
        t0 = time.perf_counter()
        bm.prepare_prefill_metadata(slots, lens, [0] * 32, [[] for _ in slots])
        pack_times.append(time.perf_counter() - t0)
        for s_ in slots:
            bm.free_slot(s_)
    pack_s = sorted(pack_times[3:])[2]
    return {
        "cores": cores, "kind": "port",
        "decode_4seq": {"us": round(dec_s * 1e6, 1), "gbs": round(nbytes / dec_s / 1e9, 2),
                        "sample": "fp32 torch-CPU oracle, layer 0, median of 20 after 3 warm-ups"},
        "pack_prefill_32_prompts": {"us": round(pack_s * 1e6, 1), "tokens": t,
                                    "sample": "oracle block manager (per-token slot loop), median of 5"},
        "prefill_32xU64-2048": {"ms": round(pf_s * 1e3, 1),
                                "tflops": round(W.causal_attention_flops(lens, lens, 16) / pf_s / 1e12, 3),
                                "sample": f"fp32 torch-CPU oracle, median of {prefill_reps} after 3 warm-ups"},
        "kv_write_32xU64-2048": {"ms": round(kv_s * 1e3, 2), "bytes": kv_bytes,
                                 "gbs": round(kv_bytes / kv_s / 1e9, 2),
                                 "sample": "torch-CPU index_copy_ of the prompts' bf16 K and V into a 1024 x 128-token "
                                           "block cache through the slot mapping (the reference's PagedKVCache.write), "
                                           "median of 20 after 3 warm-ups"},
    }


def cpu_e2e_truncated(state, config, prompts: list[list[int]], n_decode: int, workload: str) -> dict:
    """fp32 oracle model on the host cores (oracle/qwen3_ref.py: one sequence at a time, dense cache,
    the same weights) over a truncated run: each prompt's prefill, then `n_decode` greedy decode steps."""
    import torch

    from oracle.qwen3_ref import Qwen3Ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ref = Qwen3Ref(state, config, round_bf16=True, max_positions=max(len(p) for p in prompts) + n_decode + 1)
    t_prefill = t_decode = 0.0
    for prompt in prompts:
        ref.reset()
        t0 = time.perf_counter()
        tok = int(ref.forward(prompt).argmax())
        t_prefill += time.perf_counter() - t0
        t0 = time.perf_counter()
        for _ in range(n_decode):
            tok = int(ref.forward([tok]).argmax())
        t_decode += time.perf_counter() - t0
    steps = len(prompts) * n_decode
    return {"truncated": True, "kind": "port", "cores": cores, "cpu": cpu_model(),
            "sample": f"{workload}: {len(prompts)} of its prompts, each prefilled then {n_decode} greedy decode steps, "
                      f"one sequence at a time (fp32 CPU oracle model, same weights)",
            "prefill_tok_s": round(sum(len(p) for p in prompts) / t_prefill, 2),
            "decode_tok_s": round(steps / t_decode, 3), "decode_step_ms": round(t_decode / steps * 1e3, 1)}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards by sequence, or by kv head with one o_proj all-reduce per layer; only the "
              "one-GPU share is built and measured)", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    device = torch.device("cuda:0")
    torch.manual_seed(args.seed)

    dec = decode_leg(args, device)
    workload = "decode_b32_ctx256-2304_28layers"
    traffic, traffic_source = load_traffic(workload)
    result = {
        "metric": "paged decode-attn HBM GB/s (% of peak); Qwen3-0.6B output tok/s 32x256/2048",
        "value": round(dec["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/K/V, seeded context lengths and block tables)",
        "config": {
            "workload": workload,
            "batch": 32,
            "context_lens": "uniform [256, 2304], seed %d" % args.seed,
            "sum_context": sum(dec["work"].context_lens_list),
            "layers_per_step": NUM_LAYERS,
            "num_heads": 16,
            "num_kv_heads": 8,
            "head_dim": 128,
            "block_size": 128,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_decode_kernel",
            "achieved": round(dec["achieved"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["achieved"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "bytes_per_launch": dec["bytes_per_launch"],
            "avg_launch_us": round(dec["avg_launch_us"], 3),
            "median_launch_us": round(dec["median_launch_us"], 3),
        },
    }
    result["fused_step"] = fused_step_leg(args, dec["work"], device)
    result["pack"] = pack_leg(args, device)
    small = small_decode_leg(args, device)
    result["decode_small"] = {k: v for k, v in small.items() if k != "work"}
    result["decode_scaling"] = decode_scaling_leg(args, device)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(dec["work"], args.seed)
        result["cpu_baseline_other"] = cpu_baselines_other(small["work"], args.seed)
    del dec, small
    torch.cuda.empty_cache()
    if not args.no_prefill:
        result["prefill"] = prefill_leg(args, device)
        torch.cuda.empty_cache()
    if not args.no_e2e:
        try:
            from nano_vllm_ascend_amd.bench_e2e import run_e2e
        except ImportError:
            run_e2e = None
        if run_e2e is not None:
            from nano_vllm_ascend_amd import LLM
            from nano_vllm_ascend_amd.bench_e2e import make_dataset
            from nano_vllm_ascend_amd.config import QWEN3_0_6B

            cfg = QWEN3_0_6B
            need = args.e2e_prompts * -(-(args.e2e_input + args.e2e_output) // 128)
            llm = LLM(cfg, max_model_len=4096, num_blocks=need + 64, max_num_seqs=args.e2e_prompts, seed=args.seed)
            e2e = run_e2e(args.e2e_prompts, args.e2e_input, args.e2e_output, seed=args.seed, llm=llm)
            e2e["vs_reference_910B3"] = round(e2e["output_tok_s"] / REFERENCE_E2E_TOK_S, 3)
            result["e2e"] = e2e
            state = None
            if not args.no_cpu:
                state = {k: v.detach().to("cpu") for k, v in llm.runner.model.state_dict().items()}
            del llm
            torch.cuda.empty_cache()
            if not args.no_load:
                load = run_e2e(100, 2048, args.load_output, seed=args.seed, shared_prefix=1024, shared_fraction=0.5,
                               enable_prefix_cache=True, graph_sizes=[1, 2, 4, 8, 16, 32, 64, 100])
                load["vs_reference_910B3"] = round(load["output_tok_s"] / REFERENCE_LOAD_TOK_S, 3)
                load["reference_note"] = ("the reference's 100 x 2048/2048 run (1410.2 output tok/s, batch-100 graph) "
                                          "used random prompts without a shared prefix")
                result["e2e_load"] = load
                torch.cuda.empty_cache()
            if state is not None:
                p3 = make_dataset(args.e2e_prompts, args.e2e_input, cfg.vocab_size, args.seed)[:2]
                p4 = make_dataset(100, 2048, cfg.vocab_size, args.seed, shared_prefix=1024, shared_fraction=0.5)[:1]
                result["cpu_baseline_e2e"] = {
                    "32x256/2048": cpu_e2e_truncated(state, cfg, p3, 32, "32 x 256/2048"),
                    "100x2048/2048": cpu_e2e_truncated(state, cfg, p4, 32, "100 x 2048/2048"),
                }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
