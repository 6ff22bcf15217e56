"""The allocation-free decode entry point equals the workspace one, bit for bit.

nvamd_paged_decode_noalloc uses the library's static per-GPU scratch instead
of a caller's workspace.  Two calls in a row (the second smaller, so it finds
the first call's leftovers in the shared scratch) must each equal
nvamd_paged_decode with a fresh workspace on the same inputs, and a call that
needs more than the scratch holds is refused before anything is launched.
"""
from __future__ import annotations

import pytest
import torch

from nano_vllm_ascend_amd import _C
from nano_vllm_ascend_amd import workloads as W

SCALE = 128 ** -0.5


def _both(work, bound, device):
    q, kc, vc = work.q, work.key_cache[0], work.value_cache[0]
    want = torch.empty_like(q)
    ws = _C.alloc_paged_decode_workspace(q.shape[0], 16, 8, bound, device)
    _C.paged_decode(want, q, kc, vc, work.block_tables, work.context_lens, SCALE, bound, ws)
    got = torch.full_like(q, float("nan"))
    _C.paged_decode_noalloc(got, q, kc, vc, work.block_tables, work.context_lens, SCALE, bound)
    torch.cuda.synchronize()
    return got, want


@pytest.mark.gpu
def test_noalloc_decode_captured_in_a_graph_equals_workspace_decode(device):
    """Graph capture is what the entry point is for.  The first call on a device clears the scratch's
    counters, so it is refused under capture (ValueError, nothing recorded); once a call ran eagerly,
    a captured call replays correctly, with eager calls in between, and with new q values."""
    work = W.decode_step(device, seed=6)
    q, kc, vc = work.q, work.key_cache[0], work.value_cache[0]
    got = torch.full_like(q, float("nan"))
    args = (kc, vc, work.block_tables, work.context_lens, SCALE, 2304)
    g = torch.cuda.CUDAGraph()
    try:  # refused only if no call has set the device up yet (this test runs first in its file)
        with torch.cuda.graph(g):
            _C.paged_decode_noalloc(got, q, *args)
        refused = False
    except ValueError as e:
        assert "graph capture" in str(e)
        refused = True
    print(f"[no-alloc] first capture refused: {refused}", flush=True)
    torch.cuda.synchronize()
    if refused:
        _C.paged_decode_noalloc(got, q, *args)  # eager: sets the device up
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            _C.paged_decode_noalloc(got, q, *args)
    ws = _C.alloc_paged_decode_workspace(q.shape[0], 16, 8, 2304, device)
    for rep in range(3):
        if rep == 2:
            q.mul_(-0.5)  # the graph reads q in place
        want = torch.empty_like(q)
        _C.paged_decode(want, q, *args[:-1], 2304, ws)
        got.fill_(float("nan"))
        small = W.make_decode(4, 1, 512, 64, seed=rep, device=device)  # an eager call between replays
        other = torch.empty_like(small.q)
        _C.paged_decode_noalloc(other, small.q, small.key_cache[0], small.value_cache[0], small.block_tables,
                                small.context_lens, SCALE, 4096)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), rep


@pytest.mark.gpu
def test_noalloc_decode_equals_workspace_decode_on_two_calls(device):
    # first: 32 sequences of U[256, 2304] (split-KV launches: the counters and partials are used)
    big = W.decode_step(device, seed=3)
    print(f"[no-alloc] call 1: batch {len(big.context_lens_list)}, contexts up to {max(big.context_lens_list)}",
          flush=True)
    got, want = _both(big, 2304, device)
    assert torch.equal(got, want)
    # second, smaller: 4 sequences of U[1, 512] with a 4096-token bound (still split-KV)
    small = W.make_decode(4, 1, 512, 64, seed=4, device=device)
    print(f"[no-alloc] call 2: batch 4, contexts {small.context_lens_list}", flush=True)
    got, want = _both(small, 4096, device)
    assert torch.equal(got, want)
    # and the first shape again: the counters were left at zero by the calls before
    got, want = _both(big, 2304, device)
    assert torch.equal(got, want)


@pytest.mark.gpu
def test_noalloc_decode_refuses_sizes_beyond_the_scratch(device):
    work = W.make_decode(4, 1, 512, 64, seed=5, device=device)
    bound = 2_621_440  # 4 rows x 8 kv heads x 2 GQA rows of partials per 256 tokens: 346 MB > 64 MiB
    assert _C.paged_decode_workspace_size(4, 16, 8, bound) > _C.DECODE_SCRATCH_BYTES
    out = torch.zeros_like(work.q)
    with pytest.raises(ValueError, match="static scratch"):
        _C.paged_decode_noalloc(out, work.q, work.key_cache[0], work.value_cache[0], work.block_tables,
                                work.context_lens, SCALE, bound)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0  # nothing was launched
