"""Parity of the HIP paged decode kernel with the fp32 oracle (max-abs <= 2e-2 in bf16)."""
from __future__ import annotations

import pytest
import torch

from nano_vllm_ascend_amd import _C
from nano_vllm_ascend_amd import workloads as W
from oracle.attention_ref import paged_decode_ref

TOL = 2e-2  # max-abs error allowed against the fp32 reference of the same paged semantics
SCALE = W.HEAD_DIM ** -0.5


def run_decode(q, kc, vc, block_tables, context_lens, max_ctx, out=None, ws=None):
    out = torch.empty_like(q) if out is None else out
    if ws is None:
        ws = _C.alloc_paged_decode_workspace(q.shape[0], q.shape[1], kc.shape[2], max_ctx, q.device)
    _C.paged_decode(out, q, kc, vc, block_tables, context_lens, SCALE, max_ctx, ws)
    return out


def check(work, layer=0, max_ctx=None):
    max_ctx = max_ctx or max(work.context_lens_list)
    out = run_decode(work.q, work.key_cache[layer], work.value_cache[layer], work.block_tables,
                     work.context_lens, max_ctx)
    torch.cuda.synchronize()
    ref = paged_decode_ref(work.q, work.key_cache[layer], work.value_cache[layer], work.block_tables,
                           work.context_lens, SCALE)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL, f"max-abs {err:.4g} > {TOL}"
    return err


@pytest.mark.gpu
def test_decode_single_layer_batch4(device):
    for seed in range(3):
        check(W.decode_single(device, seed=seed))


@pytest.mark.gpu
def test_decode_step_batch32(device):
    work = W.decode_step(device, seed=0)
    check(work)
    # a larger bound than needed only adds empty workgroups
    check(work, max_ctx=4096)


@pytest.mark.gpu
@pytest.mark.parametrize("ctx", [1, 2, 15, 16, 17, 127, 128, 129, 255, 256, 257, 511, 512, 513, 1023, 1024, 1025,
                                 2047, 2048, 2049, 4096])
def test_decode_edge_lengths(device, ctx):
    work = W.make_decode(3, 0, 0, 160, seed=ctx, device=device, context_lens=[ctx, max(1, ctx // 3), 1])
    check(work)


@pytest.mark.gpu
def test_decode_long_contexts_many_partitions(device):
    """Contexts of 4200-9000 tokens: up to 36 partitions per (sequence, kv head), past the 16 the
    merge loads in its first round, so later partitions arrive 8 per round."""
    work = W.make_decode(8, 4200, 9000, 600, seed=17, device=device)
    assert max(work.context_lens_list) > 16 * 256
    check(work)
    check(work, max_ctx=12000)  # a looser bound only adds empty workgroups


@pytest.mark.gpu
@pytest.mark.parametrize("lo,hi,seed", [(16400, 32000, 23), (33000, 40960, 29)])
def test_decode_very_long_contexts_several_chunks_per_wave(device, lo, hi, seed):
    """Bounds past 64 partitions of 256 tokens (16,384 tokens) give each wave two 64-token chunks,
    bounds past 32,768 tokens four; the second case reaches Qwen3's 40,960 positions."""
    work = W.make_decode(2, lo, hi, 2 * (hi // 128 + 1), seed=seed, device=device)
    assert max(work.context_lens_list) > 16384
    check(work)
    check(work, max_ctx=40960)  # the four-chunk launch over shorter contexts


@pytest.mark.gpu
def test_decode_at_the_two_chunk_boundary(device):
    """Bounds of 16,384 and 16,385 tokens take one and two chunks per wave; contexts at and around
    the boundary, and short ones, give the same results under both."""
    work = W.make_decode(4, 0, 0, 4 * 129, seed=37, device=device, context_lens=[16384, 16383, 16385, 300])
    a = check(work, max_ctx=16385)
    short = W.make_decode(3, 0, 0, 3 * 129, seed=38, device=device, context_lens=[16384, 1, 7000])
    check(short, max_ctx=16384)
    check(short, max_ctx=16385)
    assert a <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["ramp", "large"])
def test_decode_partitions_with_far_apart_maxima(device, case):
    """Keys scaled up along each context (ramp: later partitions' maxima exceed earlier ones by tens
    of log2 units, so the merge weighs early partitions by ~0 and the running maximum moves inside
    partitions) or large everywhere (q and k ~ N(0, 9))."""
    work = W.make_decode(8, 1000, 3000, 200, seed=31, device=device)
    bs = work.key_cache.shape[2]
    if case == "ramp":
        for i, n in enumerate(work.context_lens_list):
            pos = torch.arange(n, device=device)
            blocks = work.block_tables[i, pos // bs].long()
            gain = (1.0 + pos.float() / 64.0)[:, None, None]
            rows = work.key_cache[0, blocks, pos % bs].float()
            work.key_cache[0, blocks, pos % bs] = (rows * gain).to(torch.bfloat16)
    else:
        work.key_cache[0].mul_(3.0)
        work.q.mul_(3.0)
    check(work)


@pytest.mark.gpu
def test_decode_large_ragged_batch_with_empty_sequences(device):
    """150 sequences (the work list spans three 64-sequence scans), some with no context."""
    gen = torch.Generator().manual_seed(21)
    ctx = torch.randint(0, 1500, (150,), generator=gen).tolist()
    for i in (0, 63, 64, 100, 149):
        ctx[i] = 0
    ctx[1], ctx[65] = 1, 1499
    work = W.make_decode(150, 0, 0, 1400, seed=21, device=device, context_lens=ctx)
    out_tight = run_decode(work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens,
                           max(ctx))
    check(work, max_ctx=4096)
    torch.cuda.synchronize()
    assert int(out_tight[[0, 63, 64, 100, 149]].abs().sum()) == 0  # empty sequences give zeros
    ref = paged_decode_ref(work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens,
                           SCALE)
    assert (out_tight.float().cpu() - ref).abs().max().item() <= TOL


# (24, 8), (40, 8) and (32, 4): ratios 3, 5 and 8 (Qwen3-14B and -32B have 5 and 8) run as several
# launches over 4, 2 and 1 query heads of every kv head.
GQA_HEADS = [(8, 8), (16, 8), (16, 4), (24, 8), (40, 8), (32, 4)]


@pytest.mark.gpu
@pytest.mark.parametrize("heads", GQA_HEADS)
def test_decode_gqa_groups(device, heads):
    hq, hkv = heads
    work = W.make_decode(5, 1, 700, 64, seed=7, device=device, num_heads=hq, num_kv_heads=hkv)
    check(work)


@pytest.mark.gpu
@pytest.mark.parametrize("bs", [16, 32, 64, 256])
def test_decode_block_sizes(device, bs):
    work = W.make_decode(4, 1, 600, 256, seed=bs, device=device, block_size=bs)
    check(work)


@pytest.mark.gpu
@pytest.mark.parametrize("heads", GQA_HEADS)
@pytest.mark.parametrize("bs", [16, 128])
def test_decode_split_path_gqa_and_block_sizes(device, heads, bs):
    """Batches large enough for the split-KV launch (nontemporal loads, cross-workgroup merge)
    at every GQA group and a small and a large block size; the small-batch tests above take
    the whole-unit launch."""
    hq, hkv = heads
    work = W.make_decode(48, 300, 900, 48 * 900 // bs + 8, seed=bs + hq, device=device, block_size=bs,
                         num_heads=hq, num_kv_heads=hkv)
    assert 48 * hkv * -(-max(work.context_lens_list) // 256) >= 2 * 256  # split launch on a 256-CU GPU
    check(work)


@pytest.mark.gpu
def test_decode_ignores_stale_rows_past_context(device):
    """Unwritten rows of the last block may hold NaN bit patterns; they must not reach the output."""
    work = W.make_decode(4, 1, 300, 16, seed=3, device=device)
    bs = work.key_cache.shape[2]
    bt = work.block_tables.cpu()
    for i, c in enumerate(work.context_lens_list):
        last = int(bt[i, (c - 1) // bs])
        off = c % bs
        if off:
            work.key_cache[0, last, off:] = float("nan")
            work.value_cache[0, last, off:] = float("inf")
    err = check(work)
    assert err == err  # not NaN


@pytest.mark.gpu
def test_decode_workspace_reused_across_shapes(device):
    """Counters are left at zero, so one workspace serves calls of different batch and bound."""
    big = W.decode_step(device, seed=1)
    small = W.decode_single(device, seed=1)
    ws = _C.alloc_paged_decode_workspace(32, 16, 8, 4096, device)
    for _ in range(2):
        for work, mc in ((big, 4096), (small, 512), (big, 2304)):
            out = run_decode(work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens,
                             mc, ws=ws)
            torch.cuda.synchronize()
            ref = paged_decode_ref(work.q, work.key_cache[0], work.value_cache[0], work.block_tables,
                                   work.context_lens, SCALE)
            assert (out.float().cpu() - ref).abs().max().item() <= TOL
    counters = ws[: 16384 * 4].view(torch.int32)
    assert int(counters.abs().sum()) == 0


@pytest.mark.gpu
def test_decode_strided_query_view(device):
    """q may be a view into a fused [B, (Hq+2Hkv)*D] projection; out may be strided too."""
    work = W.decode_single(device, seed=5)
    b = work.q.shape[0]
    qkv = torch.zeros(b, 32 * 128, dtype=torch.bfloat16, device=device)
    qkv[:, : 16 * 128] = work.q.reshape(b, -1)
    qv = qkv[:, : 16 * 128].view(b, 16, 128)
    outbuf = torch.zeros(b, 24 * 128, dtype=torch.bfloat16, device=device)
    outv = outbuf[:, 8 * 128 :].view(b, 16, 128)
    run_decode(qv, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens, 512, out=outv)
    torch.cuda.synchronize()
    ref = paged_decode_ref(work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens,
                           SCALE)
    assert (outv.float().cpu() - ref).abs().max().item() <= TOL
    assert int(outbuf[:, : 8 * 128].abs().sum()) == 0  # nothing written outside the view


@pytest.mark.gpu
def test_decode_graph_replays_read_device_context_lens(device):
    """A captured launch replays with new context_lens / q / tables and no host-side update."""
    work = W.decode_step(device, seed=2)
    b = work.q.shape[0]
    q = work.q.clone()
    bt = work.block_tables.clone()
    cl = work.context_lens.clone()
    out = torch.empty_like(q)
    ws = _C.alloc_paged_decode_workspace(b, 16, 8, 4096, device)
    kc, vc = work.key_cache[0], work.value_cache[0]
    run_decode(q, kc, vc, bt, cl, 4096, out=out, ws=ws)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_decode(q, kc, vc, bt, cl, 4096, out=out, ws=ws)
    gen = torch.Generator().manual_seed(11)
    for rep in range(4):
        new_ctx = torch.randint(1, 2305, (b,), generator=gen, dtype=torch.int32)
        new_ctx = torch.minimum(new_ctx, torch.tensor(work.context_lens_list, dtype=torch.int32))
        cl.copy_(new_ctx.to(device))
        q.copy_(torch.randn(q.shape, generator=gen).to(torch.bfloat16).to(device))
        graph.replay()
        torch.cuda.synchronize()
        ref = paged_decode_ref(q, kc, vc, bt, cl, SCALE)
        err = (out.float().cpu() - ref).abs().max().item()
        assert err <= TOL, f"replay {rep}: {err}"
        eager = run_decode(q, kc, vc, bt, cl, 4096, ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(eager, out), f"replay {rep} differs from eager"


@pytest.mark.gpu
def test_range_checks_raise_before_launching(device):
    """With range checks on, indices the reference's indexing would reject raise IndexError from the
    eager wrappers (nothing is launched); in-range calls run as usual."""
    from nano_vllm_ascend_amd.layers import RotaryEmbedding

    work = W.make_decode(4, 1, 512, 64, seed=6, device=device)
    q, kc, vc = work.q, work.key_cache[0], work.value_cache[0]
    ws = _C.alloc_paged_decode_workspace(4, 16, 8, 512, device)
    out = torch.zeros_like(q)
    prev = _C.set_range_checks(True)
    try:
        _C.paged_decode(out, q, kc, vc, work.block_tables, work.context_lens, 128 ** -0.5, 512, ws)
        too_long = work.context_lens.clone()
        too_long[0] = work.block_tables.shape[1] * 128 + 1
        with pytest.raises(IndexError):
            _C.paged_decode(out, q, kc, vc, work.block_tables, too_long, 128 ** -0.5, 4096, ws)
        k = torch.randn(2, 8, 128, device=device).bfloat16()
        with pytest.raises(IndexError):
            _C.kv_cache_write(k, k, kc, vc, torch.tensor([0, kc.shape[0] * 128], device=device))
        table = RotaryEmbedding(128, 1024, 1e6).cos_sin.to(device)
        qq = torch.randn(2, 16, 128, device=device).bfloat16()
        with pytest.raises(IndexError):
            _C.qk_norm_rope(qq, k.clone(), torch.ones(128, device=device).bfloat16(),
                            torch.ones(128, device=device).bfloat16(), torch.tensor([3, 1024], device=device), table,
                            1e-6)
    finally:
        _C.set_range_checks(prev)
    torch.cuda.synchronize()
