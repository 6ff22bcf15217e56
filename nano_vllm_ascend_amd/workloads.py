"""Seeded synthetic workloads at the shapes the attention path is measured on.

Qwen3-0.6B attention shape: 16 query heads, 8 KV heads (GQA 2), head_dim 128,
block_size 128, bf16.  Lengths come from ``random.Random(seed)``; tensors from
a ``torch.Generator`` seeded with the same seed.

decode_single    one paged decode attention: batch 4, context lengths
                 uniform in [1, 512], block tables drawn from a seeded
                 permutation of a 64-block pool, q/K/V ~ N(0, 1).
decode_step      one decode step of 32 sequences with context lengths uniform
                 in [256, 2304] (the new token sits at position ctx-1): fused
                 qkv activations [32, 4096] ~ N(0, 1), q/k norm weights
                 ~ N(1, 0.02), pool a seeded permutation of >= 1024 blocks.
ragged_prefill   32 prompts, lengths uniform in [64, 2048], packed with
                 cu_seqlens; q/k/v ~ N(0, 1).
"""
from __future__ import annotations

import math
import random
from dataclasses import dataclass

import torch

NUM_HEADS = 16
NUM_KV_HEADS = 8
HEAD_DIM = 128
BLOCK_SIZE = 128
ROPE_THETA = 1.0e6
RMS_EPS = 1.0e-6


@dataclass
class PagedBatch:
    context_lens: list[int]
    block_tables: torch.Tensor  # int32 [B, W]
    num_blocks: int
    block_size: int


def seeded_block_tables(context_lens: list[int], num_blocks: int, block_size: int, seed: int,
                        width: int | None = None) -> PagedBatch:
    """Give each sequence ceil(ctx/bs) distinct blocks, taken in order from a seeded permutation of the pool."""
    need = [max(1, math.ceil(c / block_size)) for c in context_lens]
    if sum(need) > num_blocks:
        raise ValueError(f"pool of {num_blocks} blocks cannot hold {sum(need)}")
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    w = width or max(need)
    tables = torch.zeros(len(context_lens), w, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(need):
        tables[i, :n] = torch.tensor(perm[pos : pos + n], dtype=torch.int32)
        pos += n
    return PagedBatch(list(context_lens), tables, num_blocks, block_size)


def _randn(shape, gen, device, dtype=torch.bfloat16, mean=0.0, std=1.0):
    t = torch.empty(shape, dtype=torch.float32, device=device)
    t.normal_(mean, std, generator=gen)
    return t.to(dtype)


def _generator(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


@dataclass
class DecodeWorkload:
    q: torch.Tensor            # [B, Hq, D] bf16
    key_cache: torch.Tensor    # [L, NB, bs, Hkv, D] bf16
    value_cache: torch.Tensor
    block_tables: torch.Tensor  # int32 [B, W] on device
    context_lens: torch.Tensor  # int32 [B] on device
    context_lens_list: list[int]
    num_layers: int

    @property
    def num_blocks(self) -> int:
        return self.key_cache.shape[1]


def decode_lengths(batch: int, lo: int, hi: int, seed: int) -> list[int]:
    rng = random.Random(seed)
    return [rng.randint(lo, hi) for _ in range(batch)]


def make_decode(batch: int, ctx_lo: int, ctx_hi: int, num_blocks: int, seed: int, device,
                num_layers: int = 1, block_size: int = BLOCK_SIZE, num_heads: int = NUM_HEADS,
                num_kv_heads: int = NUM_KV_HEADS, context_lens: list[int] | None = None,
                width: int | None = None) -> DecodeWorkload:
    ctx = context_lens or decode_lengths(batch, ctx_lo, ctx_hi, seed)
    pb = seeded_block_tables(ctx, num_blocks, block_size, seed, width)
    gen = _generator(device, seed)
    q = _randn((len(ctx), num_heads, HEAD_DIM), gen, device)
    shape = (num_layers, num_blocks, block_size, num_kv_heads, HEAD_DIM)
    kc = _randn(shape, gen, device)
    vc = _randn(shape, gen, device)
    return DecodeWorkload(q, kc, vc, pb.block_tables.to(device), torch.tensor(ctx, dtype=torch.int32, device=device),
                          list(ctx), num_layers)


def decode_single(device, seed: int = 0, num_layers: int = 1) -> DecodeWorkload:
    """Batch 4, context U[1, 512], 64-block pool."""
    return make_decode(4, 1, 512, 64, seed, device, num_layers=num_layers)


def decode_step_lengths(seed: int = 0) -> list[int]:
    return decode_lengths(32, 256, 2304, seed)


def decode_step(device, seed: int = 0, num_layers: int = 1, num_blocks: int = 1024) -> DecodeWorkload:
    """Batch 32, context U[256, 2304], 1024-block pool."""
    return make_decode(32, 256, 2304, num_blocks, seed, device, num_layers=num_layers)


@dataclass
class FusedStepInputs:
    qkv: torch.Tensor        # [B, (Hq + 2 Hkv) * D] bf16, the fused projection output
    q_weight: torch.Tensor   # [D] bf16
    k_weight: torch.Tensor   # [D] bf16
    positions: torch.Tensor  # int64 [B] = ctx - 1
    slot_mapping: torch.Tensor  # int64 [B]


def fused_step_inputs(work: DecodeWorkload, seed: int, device) -> FusedStepInputs:
    """Activations of one decode step over `work`: the new token of sequence i is at ctx_i - 1."""
    gen = _generator(device, seed + 1)
    b = len(work.context_lens_list)
    qkv = _randn((b, (NUM_HEADS + 2 * NUM_KV_HEADS) * HEAD_DIM), gen, device)
    qw = _randn((HEAD_DIM,), gen, device, mean=1.0, std=0.02)
    kw = _randn((HEAD_DIM,), gen, device, mean=1.0, std=0.02)
    bs = work.key_cache.shape[2]
    bt = work.block_tables.cpu()
    pos = [c - 1 for c in work.context_lens_list]
    slots = [int(bt[i, p // bs]) * bs + p % bs for i, p in enumerate(pos)]
    return FusedStepInputs(qkv, qw, kw, torch.tensor(pos, dtype=torch.int64, device=device),
                           torch.tensor(slots, dtype=torch.int64, device=device))


def prefill_lengths(num_seqs: int = 32, lo: int = 64, hi: int = 2048, seed: int = 0) -> list[int]:
    rng = random.Random(seed)
    return [rng.randint(lo, hi) for _ in range(num_seqs)]


def causal_attention_flops(q_lens, kv_lens, num_heads: int, head_dim: int = 128) -> float:
    """Algorithmic FLOPs of causal (bottom-right) attention: 4 * head_dim * num_heads per visible
    (query, key) pair, QK^T and PV; query row r of a sequence sees kv_len - q_len + r + 1 keys."""
    pairs = 0
    for ql, kl in zip(q_lens, kv_lens):
        pairs += ql * (kl - ql) + ql * (ql + 1) // 2
    return 4.0 * head_dim * num_heads * pairs


def cu_seqlens(lengths: list[int]) -> list[int]:
    out = [0]
    for n in lengths:
        out.append(out[-1] + n)
    return out
