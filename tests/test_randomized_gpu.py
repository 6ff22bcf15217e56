"""Seeded random shapes through the attention kernels, against the fp32 oracle.

Each case draws a batch size, context or prompt lengths (with lengths on block and partition
edges mixed in), a GQA ratio, a block size and a context bound looser than the longest context,
so the launch kinds (whole-unit and split decode, several launches per group for ratios other
than 1, 2 and 4, dense and paged prefill) meet shapes the fixed tests do not pin.  The cases are
the same on every run (random.Random(seed)).
"""
from __future__ import annotations

import math
import random

import pytest
import torch

from nano_vllm_ascend_amd import _C
from nano_vllm_ascend_amd import workloads as W
from oracle.attention_ref import paged_decode_ref, paged_prefill_ref, varlen_prefill_ref

from test_fused_decode_gpu import Case, check as check_fused

TOL = 2e-2
SCALE = W.HEAD_DIM ** -0.5
HEADS = [(8, 8), (16, 8), (24, 8), (16, 4), (40, 8), (32, 4), (4, 1)]
EDGES = [1, 2, 15, 16, 17, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512, 513]


def _lengths(rng: random.Random, n: int, hi: int) -> list[int]:
    out = []
    for _ in range(n):
        out.append(rng.choice(EDGES) if rng.random() < 0.3 else rng.randint(1, hi))
    return out


def _decode_case(seed: int, device):
    rng = random.Random(seed)
    batch = rng.choice([1, 3, 8, 33, 70])
    hq, hkv = rng.choice(HEADS)
    bs = rng.choice([16, 32, 64, 128, 256])
    ctx = _lengths(rng, batch, rng.choice([600, 3000]))
    bound = max(ctx) + rng.choice([0, 1, 200])
    num_blocks = sum(math.ceil(c / bs) for c in ctx) + 4
    work = W.make_decode(batch, 0, 0, num_blocks, seed, device, block_size=bs, num_heads=hq, num_kv_heads=hkv,
                         context_lens=ctx, width=math.ceil(bound / bs))
    return work, bound, (batch, hq, hkv, bs, bound)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(12))
def test_random_decode_shapes(device, seed):
    work, bound, desc = _decode_case(seed, device)
    print(f"decode case {seed}: batch, hq, hkv, block, bound = {desc}", flush=True)
    out = torch.empty_like(work.q)
    ws = _C.alloc_paged_decode_workspace(work.q.shape[0], work.q.shape[1], work.key_cache.shape[3], bound, device)
    _C.paged_decode(out, work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens, SCALE,
                    bound, ws)
    torch.cuda.synchronize()
    ref = paged_decode_ref(work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens, SCALE)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL, (desc, err)
    # a second call on the same workspace (its counters were left at zero) gives the same bits
    out2 = torch.empty_like(out)
    _C.paged_decode(out2, work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens,
                    SCALE, bound, ws)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), desc


def _rand(shape, gen, device):
    return torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(8))
def test_random_prefill_shapes(device, seed):
    rng = random.Random(1000 + seed)
    n = rng.choice([1, 2, 5, 9])
    hq, hkv = rng.choice(HEADS)
    lens = _lengths(rng, n, rng.choice([300, 900]))
    print(f"prefill case {seed}: prompts {lens}, heads {hq}/{hkv}", flush=True)
    gen = torch.Generator(device=device).manual_seed(seed)
    t = sum(lens)
    q, k, v = _rand((t, hq, 128), gen, device), _rand((t, hkv, 128), gen, device), _rand((t, hkv, 128), gen, device)
    cu = W.cu_seqlens(lens)
    cu_dev = torch.tensor(cu, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    _C.varlen_prefill(out, q, k, v, cu_dev, max(lens), SCALE)
    torch.cuda.synchronize()
    ref = varlen_prefill_ref(q, k, v, cu, SCALE)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL, (lens, hq, hkv, err)

    # the paged route over the same prompts, each with a random cached prefix of whole blocks
    bs = rng.choice([16, 64, 128])
    nblk = [math.ceil(x / bs) for x in lens]
    num_blocks = sum(nblk) + 2
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    tables = torch.zeros(n, max(nblk), dtype=torch.int32)
    pos = 0
    for i, nb in enumerate(nblk):
        tables[i, :nb] = torch.tensor(perm[pos: pos + nb])
        pos += nb
    kc = torch.zeros((num_blocks, bs, hkv, 128), dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([int(tables[i, p // bs]) * bs + p % bs for i, x in enumerate(lens) for p in range(x)],
                         dtype=torch.int64, device=device)
    _C.kv_cache_write(k, v, kc, vc, slots)
    cached = [bs * rng.randint(0, (x - 1) // bs) for x in lens]
    sel = torch.tensor([cu[i] + p for i, x in enumerate(lens) for p in range(cached[i], x)], device=device)
    qs = q[sel].contiguous()
    q_lens = [x - c for x, c in zip(lens, cached)]
    cu_q = W.cu_seqlens(q_lens)
    outp = torch.empty_like(qs)
    _C.paged_prefill(outp, qs, kc, vc, tables.to(device), torch.tensor(cu_q, dtype=torch.int32, device=device),
                     torch.tensor(lens, dtype=torch.int32, device=device), max(q_lens), SCALE)
    torch.cuda.synchronize()
    refp = paged_prefill_ref(qs, kc, vc, tables, cu_q, lens, SCALE)
    errp = (outp.float().cpu() - refp).abs().max().item()
    assert errp <= TOL, (lens, cached, bs, hq, hkv, errp)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(6))
def test_random_fused_decode_steps(device, seed):
    """The fused decode step (norm, RoPE, KV store, attention in one launch per query-head group)
    equals the two-launch chain bit for bit and the oracle within the tolerance, on random shapes."""
    rng = random.Random(2000 + seed)
    batch = rng.choice([2, 9, 40])
    heads = rng.choice(HEADS)
    bs = rng.choice([16, 64, 128])
    ctx = _lengths(rng, batch, rng.choice([500, 2500]))
    print(f"fused case {seed}: batch {batch}, heads {heads}, block {bs}, contexts up to {max(ctx)}", flush=True)
    num_blocks = sum(math.ceil(c / bs) for c in ctx) + 4
    check_fused(Case(device, batch, 0, 0, num_blocks, seed=seed, heads=heads, bs=bs, context_lens=ctx),
                max_ctx=max(ctx) + rng.choice([0, 100]))
