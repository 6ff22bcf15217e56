"""Parity of the HIP KV store and fused QK-RMSNorm + RoPE kernels with the oracle."""
from __future__ import annotations

import pytest
import torch

from nano_vllm_ascend_amd import _C
from nano_vllm_ascend_amd import workloads as W
from oracle.attention_ref import kv_write_ref, qk_norm_rope_ref, rope_cos_sin_table

BF16_TOL = 2e-2  # max-abs; the rounding points match the reference, so most elements are bit-equal


def cos_sin_table(max_pos, device, theta=W.ROPE_THETA):
    cos, sin = rope_cos_sin_table(W.HEAD_DIM, max_pos, theta)
    return torch.cat((cos[:, :64], sin[:, :64]), dim=1).contiguous().to(device)


def random_slots(n, num_slots, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(num_slots, generator=g)[:n].to(torch.int64)


@pytest.mark.gpu
@pytest.mark.parametrize("t", [1, 7, 32, 1000])
def test_kv_cache_write_bit_exact(device, t):
    g = torch.Generator(device=device).manual_seed(t)
    nb, bs = 64, 128
    kc = torch.randn(nb, bs, 8, 128, generator=g, device=device).to(torch.bfloat16)
    vc = torch.randn(nb, bs, 8, 128, generator=g, device=device).to(torch.bfloat16)
    k = torch.randn(t, 8, 128, generator=g, device=device).to(torch.bfloat16)
    v = torch.randn(t, 8, 128, generator=g, device=device).to(torch.bfloat16)
    slots = random_slots(t, nb * bs, t)
    if t > 4:
        slots[3] = -1  # padding row: skipped
    ref_k, ref_v = kv_write_ref(k, v, kc, vc, slots)
    _C.kv_cache_write(k, v, kc, vc, slots.to(device))
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), ref_k)
    assert torch.equal(vc.cpu(), ref_v)


@pytest.mark.gpu
def test_kv_cache_write_strided_views(device):
    t = 33
    g = torch.Generator(device=device).manual_seed(1)
    qkv = torch.randn(t, 32 * 128, generator=g, device=device).to(torch.bfloat16)
    k = qkv[:, 16 * 128 : 24 * 128].view(t, 8, 128)
    v = qkv[:, 24 * 128 :].view(t, 8, 128)
    kc = torch.zeros(8, 128, 8, 128, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    slots = random_slots(t, 8 * 128, 2)
    ref_k, ref_v = kv_write_ref(k, v, kc, vc, slots)
    _C.kv_cache_write(k, v, kc, vc, slots.to(device))
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), ref_k) and torch.equal(vc.cpu(), ref_v)


def _norm_rope_case(device, t, seed, max_pos=40960):
    g = torch.Generator(device=device).manual_seed(seed)
    qkv = torch.randn(t, 32 * 128, generator=g, device=device).to(torch.bfloat16)
    qw = (1.0 + 0.02 * torch.randn(128, generator=g, device=device)).to(torch.bfloat16)
    kw = (1.0 + 0.02 * torch.randn(128, generator=g, device=device)).to(torch.bfloat16)
    pos = torch.randint(0, max_pos, (t,), generator=torch.Generator().manual_seed(seed)).to(torch.int64)
    return qkv, qw, kw, pos


@pytest.mark.gpu
@pytest.mark.parametrize("t", [1, 32, 513])
def test_qk_norm_rope_matches_reference_rounding(device, t):
    qkv, qw, kw, pos = _norm_rope_case(device, t, seed=t)
    q = qkv[:, : 16 * 128].view(t, 16, 128)
    k = qkv[:, 16 * 128 : 24 * 128].view(t, 8, 128)
    ref_q, ref_k = qk_norm_rope_ref(q.clone(), k.clone(), qw, kw, pos, W.ROPE_THETA, W.RMS_EPS, 40960)
    table = cos_sin_table(40960, device)
    _C.qk_norm_rope(q, k, qw, kw, pos.to(device), table, W.RMS_EPS)
    torch.cuda.synchronize()
    for got, ref in ((q.cpu(), ref_q), (k.cpu(), ref_k)):
        diff = (got.float() - ref.float()).abs()
        assert diff.max().item() <= BF16_TOL
        assert (diff == 0).float().mean().item() > 0.99


@pytest.mark.gpu
def test_qk_norm_rope_fused_store(device):
    work = W.decode_step(device, seed=4, num_blocks=512)
    inp = W.fused_step_inputs(work, 4, device)
    t = inp.qkv.shape[0]
    q = inp.qkv[:, : 16 * 128].view(t, 16, 128)
    k = inp.qkv[:, 16 * 128 : 24 * 128].view(t, 8, 128)
    v = inp.qkv[:, 24 * 128 :].view(t, 8, 128)
    ref_q, ref_k = qk_norm_rope_ref(q.clone(), k.clone(), inp.q_weight, inp.k_weight, inp.positions, W.ROPE_THETA,
                                    W.RMS_EPS, 40960)
    kc, vc = work.key_cache[0], work.value_cache[0]
    ref_kc, ref_vc = kv_write_ref(ref_k, v, kc, vc, inp.slot_mapping)
    table = cos_sin_table(40960, device)
    _C.qk_norm_rope(q, k, inp.q_weight, inp.k_weight, inp.positions, table, W.RMS_EPS, v=v, key_cache=kc,
                    value_cache=vc, slot_mapping=inp.slot_mapping)
    torch.cuda.synchronize()
    assert (q.cpu().float() - ref_q.float()).abs().max().item() <= BF16_TOL
    # the cache holds exactly the kernel's own post-RoPE k and the raw v
    flat_k = kc.reshape(-1, 8, 128)[inp.slot_mapping]
    flat_v = vc.reshape(-1, 8, 128)[inp.slot_mapping]
    assert torch.equal(flat_k, k) and torch.equal(flat_v, v)
    # untouched slots keep their bytes
    mask = torch.ones(kc.shape[0] * kc.shape[1], dtype=torch.bool)
    mask[inp.slot_mapping.cpu()] = False
    assert torch.equal(kc.reshape(-1, 8, 128).cpu()[mask], ref_kc.reshape(-1, 8, 128)[mask])
    assert torch.equal(vc.reshape(-1, 8, 128).cpu()[mask], ref_vc.reshape(-1, 8, 128)[mask])
