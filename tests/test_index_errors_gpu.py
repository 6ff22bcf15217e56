"""Index errors: where the reference's indexing raises, the kernels skip or clamp (no access leaves
its buffer) and set a bit in the device's error word, and the engine raises IndexError after the
step (the word travels to the host with the step's tokens, no extra synchronisation).

Reference behaviour: PagedKVCache.write's index_copy_ raises on a slot outside the cache
(nv/npu/paged_kv_cache.py:68-69); the RoPE cache lookup raises on a position past the table
(nv/layers/rotary_embedding.py:49-50); the attention ops cannot read a context longer than its
block-table row or a block outside the pool (nv/layers/npu_paged_attention.py:89-99,
nv/layers/npu_prefill_attention.py:73-96).
"""
from __future__ import annotations

import sys
from dataclasses import replace
from pathlib import Path

import pytest
import torch

from nano_vllm_ascend_amd import LLM, _C
from nano_vllm_ascend_amd import workloads as W
from nano_vllm_ascend_amd.config import QWEN3_0_6B
from oracle.attention_ref import kv_write_ref, paged_decode_ref

sys.path.insert(0, str(Path(__file__).resolve().parent))
from test_fused_decode_gpu import Case, cos_sin_table  # noqa: E402

SCALE = 128 ** -0.5


@pytest.fixture(autouse=True)
def clean_word(device):
    _C.clear_index_errors()
    torch.cuda.synchronize()
    assert _C.index_errors() == 0
    yield
    _C.clear_index_errors()
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_kv_store_skips_and_reports_a_slot_outside_the_cache(device):
    gen = torch.Generator(device=device).manual_seed(1)
    k = torch.randn(6, 8, 128, generator=gen, device=device).bfloat16()
    v = torch.randn(6, 8, 128, generator=gen, device=device).bfloat16()
    kc = torch.zeros(4, 16, 8, 128, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([3, 64, 17, -1, 5, 40], dtype=torch.int64, device=device)  # 64 slots: 64 is outside
    _C.kv_cache_write(k, v, kc, vc, slots)
    assert _C.index_errors() == _C.ERR_SLOT
    keep = slots.clone()
    keep[1] = -1  # the row the kernel skipped; -1 is padding
    ref_k, ref_v = kv_write_ref(k, v, torch.zeros_like(kc), torch.zeros_like(vc), keep)
    assert torch.equal(kc.cpu(), ref_k) and torch.equal(vc.cpu(), ref_v)
    _C.clear_index_errors()
    _C.kv_cache_write(k, v, kc, vc, keep)  # padding (-1) alone is not an error
    assert _C.index_errors() == 0


@pytest.mark.gpu
def test_norm_rope_reports_a_position_past_the_table(device):
    q = torch.randn(3, 16, 128, device=device).bfloat16()
    k = torch.randn(3, 8, 128, device=device).bfloat16()
    w = torch.ones(128, dtype=torch.bfloat16, device=device)
    table = cos_sin_table(device)[:64].contiguous()  # a 64-row RoPE table
    pos = torch.tensor([0, 63, 64], dtype=torch.int64, device=device)
    _C.qk_norm_rope(q, k, w, w, pos, table, W.RMS_EPS)
    assert _C.index_errors() == _C.ERR_POSITION


@pytest.mark.gpu
@pytest.mark.parametrize("fault", ["context", "block"])
def test_decode_reports_a_context_or_block_it_cannot_read(device, fault):
    work = W.make_decode(6, 100, 900, 64, seed=3, device=device)
    bad = 2
    ctx = list(work.context_lens_list)
    if fault == "context":
        work.context_lens[bad] = 1024  # its table row holds ctx blocks only; the bound is 1000
        want = _C.ERR_CONTEXT
    else:
        work.block_tables[bad, 0] = work.num_blocks  # one past the pool
        want = _C.ERR_BLOCK
    out = torch.empty_like(work.q)
    ws = _C.alloc_paged_decode_workspace(6, 16, 8, 1000, device)
    _C.paged_decode(out, work.q, work.key_cache[0], work.value_cache[0], work.block_tables, work.context_lens, SCALE,
                    1000, ws)
    assert _C.index_errors() == want
    # the other sequences are unaffected
    good = [i for i in range(6) if i != bad]
    ref = paged_decode_ref(work.q[good], work.key_cache[0], work.value_cache[0], work.block_tables[good].cpu(),
                           torch.tensor([ctx[i] for i in good]), SCALE)
    assert (out[good].float().cpu() - ref).abs().max().item() <= 2e-2


@pytest.mark.gpu
def test_fused_decode_reports_a_slot_outside_the_cache(device):
    case = Case(device, 4, 100, 600, 64, seed=9)
    num_slots = case.work.num_blocks * 128
    case.slots[1] = num_slots + 3
    out, kc, vc = case.fused(1024)
    assert _C.index_errors() == _C.ERR_SLOT
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_paged_prefill_reports_a_context_past_its_table_row(device):
    kc = torch.randn(8, 128, 8, 128, device=device).bfloat16()
    vc = torch.randn_like(kc)
    tables = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=device)  # rows hold 256 tokens
    q = torch.randn(20, 16, 128, device=device).bfloat16()
    cu = torch.tensor([0, 10, 20], dtype=torch.int32, device=device)
    kv_lens = torch.tensor([200, 300], dtype=torch.int32, device=device)  # 300 > 256
    out = torch.empty_like(q)
    _C.paged_prefill(out, q, kc, vc, tables, cu, kv_lens, 10, SCALE)
    assert _C.index_errors() == _C.ERR_CONTEXT


SMALL = replace(QWEN3_0_6B, num_hidden_layers=2)


@pytest.mark.gpu
@pytest.mark.parametrize("graph", [True, False])
def test_engine_raises_index_error_after_the_step_that_hit_it(device, graph):
    """A decode step whose slot mapping points outside the KV cache (planted after packing): the fused
    decode kernel skips the store and reports it, and the engine step raises IndexError when it reads
    the step's tokens.  The steps before it ran clean."""
    llm = LLM(SMALL, max_model_len=512, num_blocks=16, max_num_seqs=2, enable_decode_graph=graph, seed=0)
    llm.runner.tokenizer.eos_token_id = -1
    num_slots = llm.runner.num_blocks * llm.runner.block_size
    bm = llm.runner.block_manager
    plain, ahead = bm.prepare_decode_metadata, bm.prepare_decode_ahead
    state = {"packed": 0}

    def plant(md):
        state["packed"] += 1
        if state["packed"] == 3:  # the third decode step, packed in turn or ahead (overlapped decode)
            md.slot_mapping[0] += num_slots  # a device buffer (the graph's static one when captured)

    def planted(*args, **kwargs):
        md = plain(*args, **kwargs)
        plant(md)
        return md

    def planted_ahead(*args, **kwargs):
        packed = ahead(*args, **kwargs)
        if packed is not None:
            plant(packed[0])
        return packed

    bm.prepare_decode_metadata, bm.prepare_decode_ahead = planted, planted_ahead
    for p in ([5, 6, 7, 8], [9, 10, 11]):
        llm.submit(p, max_new_tokens=8)
    llm.step()  # prefill
    llm.step()  # decode 1
    llm.step()  # decode 2
    with pytest.raises(IndexError, match="slot_mapping entry outside the KV cache"):
        llm.step()  # decode 3: planted
    assert _C.index_errors() == 0  # the runner cleared the word when it raised
    del llm
    torch.cuda.empty_cache()
