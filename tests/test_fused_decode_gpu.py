"""Parity of the fused decode step (QK-RMSNorm + RoPE + KV store + paged decode in one launch).

The fused launch must equal the two-launch chain it replaces (qk_norm_rope with the store, then
paged_decode) bit for bit -- output and both caches -- and match the oracle composed of
qk_norm_rope_ref, kv_write_ref and paged_decode_ref within the bf16 tolerance.
"""
from __future__ import annotations

import pytest
import torch

from nano_vllm_ascend_amd import _C
from nano_vllm_ascend_amd import workloads as W
from oracle.attention_ref import kv_write_ref, paged_decode_ref, qk_norm_rope_ref, rope_cos_sin_table

BF16_TOL = 2e-2
MAX_POS = 40960


def cos_sin_table(device):
    cos, sin = rope_cos_sin_table(W.HEAD_DIM, MAX_POS, W.ROPE_THETA)
    return torch.cat((cos[:, :64], sin[:, :64]), dim=1).contiguous().to(device)


class Case:
    """A decode step: raw projection rows of the new tokens over a paged context."""

    def __init__(self, device, batch, lo, hi, num_blocks, seed, heads=(16, 8), bs=128, context_lens=None):
        hq, hkv = heads
        self.work = W.make_decode(batch, lo, hi, num_blocks, seed, device, block_size=bs, num_heads=hq,
                                  num_kv_heads=hkv, context_lens=context_lens)
        self.hq, self.hkv, self.bs = hq, hkv, bs
        g = torch.Generator(device=device).manual_seed(seed + 7)
        b = len(self.work.context_lens_list)
        self.qkv = torch.randn(b, (hq + 2 * hkv) * 128, generator=g, device=device).to(torch.bfloat16)
        self.qw = (1.0 + 0.02 * torch.randn(128, generator=g, device=device)).to(torch.bfloat16)
        self.kw = (1.0 + 0.02 * torch.randn(128, generator=g, device=device)).to(torch.bfloat16)
        bt = self.work.block_tables.cpu()
        pos = [max(c - 1, 0) for c in self.work.context_lens_list]
        self.positions = torch.tensor(pos, dtype=torch.int64, device=device)
        self.slots = torch.tensor([int(bt[i, p // bs]) * bs + p % bs for i, p in enumerate(pos)], dtype=torch.int64,
                                  device=device)
        self.table = cos_sin_table(device)

    def views(self, qkv):
        b = qkv.shape[0]
        q = qkv[:, : self.hq * 128].view(b, self.hq, 128)
        k = qkv[:, self.hq * 128 : (self.hq + self.hkv) * 128].view(b, self.hkv, 128)
        v = qkv[:, (self.hq + self.hkv) * 128 :].view(b, self.hkv, 128)
        return q, k, v

    def unfused(self, max_ctx):
        qkv = self.qkv.clone()
        q, k, v = self.views(qkv)
        kc, vc = self.work.key_cache[0].clone(), self.work.value_cache[0].clone()
        _C.qk_norm_rope(q, k, self.qw, self.kw, self.positions, self.table, W.RMS_EPS, v=v, key_cache=kc,
                        value_cache=vc, slot_mapping=self.slots)
        ws = _C.alloc_paged_decode_workspace(q.shape[0], self.hq, self.hkv, max_ctx, q.device)
        out = torch.empty_like(q)
        _C.paged_decode(out, q, kc, vc, self.work.block_tables, self.work.context_lens, 128 ** -0.5, max_ctx, ws)
        return out, kc, vc

    def fused(self, max_ctx, kc=None, vc=None, out=None, ws=None):
        q, k, v = self.views(self.qkv)
        kc = self.work.key_cache[0].clone() if kc is None else kc
        vc = self.work.value_cache[0].clone() if vc is None else vc
        ws = _C.alloc_paged_decode_workspace(q.shape[0], self.hq, self.hkv, max_ctx, q.device) if ws is None else ws
        out = torch.empty_like(q) if out is None else out
        _C.paged_decode_fused(out, q, k, v, self.qw, self.kw, self.positions, self.table, W.RMS_EPS, kc, vc,
                              self.slots, self.work.block_tables, self.work.context_lens, 128 ** -0.5, max_ctx, ws)
        return out, kc, vc

    def oracle(self):
        q, k, v = self.views(self.qkv)
        rq, rk = qk_norm_rope_ref(q.clone(), k.clone(), self.qw, self.kw, self.positions, W.ROPE_THETA, W.RMS_EPS,
                                  MAX_POS)
        kc, vc = kv_write_ref(rk, v, self.work.key_cache[0], self.work.value_cache[0], self.slots)
        return paged_decode_ref(rq, kc, vc, self.work.block_tables.cpu(), self.work.context_lens.cpu(), 128 ** -0.5)


def check(case, max_ctx=None, oracle=True):
    max_ctx = max_ctx or max(max(case.work.context_lens_list), 1)
    raw = case.qkv.clone()
    ref_out, ref_kc, ref_vc = case.unfused(max_ctx)
    out, kc, vc = case.fused(max_ctx)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out), (out.float() - ref_out.float()).abs().max().item()
    assert torch.equal(kc, ref_kc) and torch.equal(vc, ref_vc)
    assert torch.equal(case.qkv, raw)  # the projection rows are read, not rewritten
    if oracle:
        err = (out.cpu().float() - case.oracle()).abs().max().item()
        assert err <= BF16_TOL, err


@pytest.mark.gpu
def test_fused_step_batch32(device):
    """32 sequences, context U[256, 2304]: the split-KV path."""
    check(Case(device, 32, 256, 2304, 1024, seed=0))


@pytest.mark.gpu
def test_fused_step_batch4_whole_units(device):
    """4 sequences, context U[1, 512]: one workgroup per (sequence, kv head)."""
    check(Case(device, 4, 1, 512, 64, seed=1))


@pytest.mark.gpu
@pytest.mark.parametrize("heads,bs", [((8, 8), 16), ((16, 4), 64), ((16, 8), 32), ((40, 8), 128), ((32, 4), 16),
                                      ((24, 8), 64)])
def test_fused_step_gqa_and_block_sizes(device, heads, bs):
    check(Case(device, 24, 40, 1500, 4096 if bs <= 32 else 1024, seed=2, heads=heads, bs=bs))


@pytest.mark.gpu
def test_fused_step_loose_context_bound(device):
    """Graph capture passes max_model_len as the bound, not the step's longest context."""
    check(Case(device, 32, 256, 2304, 1024, seed=3), max_ctx=4096, oracle=False)


@pytest.mark.gpu
def test_fused_step_long_contexts(device):
    """Contexts past 16k tokens: several chunks per wave."""
    check(Case(device, 2, 16000, 20000, 320, seed=4))


@pytest.mark.gpu
@pytest.mark.parametrize("ctx", [1, 2, 16, 17, 128, 129, 256, 257, 1024, 1025])
def test_fused_step_edge_lengths(device, ctx):
    check(Case(device, 3, 0, 0, 64, seed=ctx, context_lens=[ctx, max(ctx - 1, 1), ctx + 5]))


@pytest.mark.gpu
def test_fused_step_token_outside_window_and_skipped_slot(device):
    """A new token past the attended context is stored but not read; slot -1 skips the store."""
    # sequence 1 owns 3 blocks (384 rows) for 301 context rows, so row 301 is its own
    case = Case(device, 6, 0, 0, 128, seed=5, context_lens=[300, 301, 555, 700, 133, 900])
    case.positions[1] = 301  # one past the context: outside the window
    bt = case.work.block_tables.cpu()
    case.slots[1] = int(bt[1, 301 // 128]) * 128 + 301 % 128
    case.slots[3] = -1
    check(case, oracle=False)


@pytest.mark.gpu
def test_fused_step_graph_replays(device):
    """A captured fused step replays with new device-side contexts, positions and slots."""
    # every row owns blocks for 1800 rows, so the replays' shorter contexts never share a block
    case = Case(device, 8, 0, 0, 256, seed=6, context_lens=[1800] * 8)
    max_ctx = 2048
    kc0, vc0 = case.work.key_cache[0].clone(), case.work.value_cache[0].clone()
    kc, vc = kc0.clone(), vc0.clone()
    ws = _C.alloc_paged_decode_workspace(8, 16, 8, max_ctx, device)
    out = torch.empty(8, 16, 128, dtype=torch.bfloat16, device=device)
    case.fused(max_ctx, kc, vc, out, ws)  # warm-up outside the graph
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        case.fused(max_ctx, kc, vc, out, ws)
    for step in range(3):
        lens = W.decode_lengths(8, 64, 1800, 100 + step)
        case.work.context_lens.copy_(torch.tensor(lens, dtype=torch.int32))
        case.work.context_lens_list = lens
        bt = case.work.block_tables.cpu()
        pos = [c - 1 for c in lens]
        case.positions.copy_(torch.tensor(pos, dtype=torch.int64))
        case.slots.copy_(torch.tensor([int(bt[i, p // 128]) * 128 + p % 128 for i, p in enumerate(pos)]))
        kc.copy_(kc0)
        vc.copy_(vc0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref_out, ref_kc, ref_vc = case.unfused(max_ctx)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out) and torch.equal(kc, ref_kc) and torch.equal(vc, ref_vc)
