"""Parity of the HIP MFMA prefill kernels with the fp32 oracle (max-abs <= 2e-2 in bf16)."""
from __future__ import annotations

import math

import pytest
import torch

from nano_vllm_ascend_amd import _C
from nano_vllm_ascend_amd import workloads as W
from oracle.attention_ref import paged_prefill_ref, varlen_prefill_ref

TOL = 2e-2
SCALE = 128 ** -0.5


def rand(shape, gen, device):
    return torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)


def run_dense(lens, hq, hkv, device, seed=0, fused=False):
    gen = torch.Generator(device=device).manual_seed(seed)
    t = sum(lens)
    if fused:  # views into one [T, (Hq + 2Hkv) * 128] projection output
        qkv = rand((t, (hq + 2 * hkv) * 128), gen, device)
        q = qkv[:, : hq * 128].view(t, hq, 128)
        k = qkv[:, hq * 128 : (hq + hkv) * 128].view(t, hkv, 128)
        v = qkv[:, (hq + hkv) * 128 :].view(t, hkv, 128)
    else:
        q, k, v = rand((t, hq, 128), gen, device), rand((t, hkv, 128), gen, device), rand((t, hkv, 128), gen, device)
    cu = W.cu_seqlens(lens)
    out = torch.empty(t, hq, 128, dtype=torch.bfloat16, device=device)
    _C.varlen_prefill(out, q, k, v, torch.tensor(cu, dtype=torch.int32, device=device), max(lens), SCALE)
    torch.cuda.synchronize()
    return out, q, k, v, cu


@pytest.mark.gpu
@pytest.mark.parametrize("lens", [[1], [5, 63, 64, 65], [1, 2, 3, 127, 128, 129, 300], [17] * 9])
def test_dense_prefill_edge_lengths(device, lens):
    out, q, k, v, cu = run_dense(lens, 16, 8, device, seed=len(lens))
    ref = varlen_prefill_ref(q, k, v, cu, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("heads", [(8, 8), (16, 4), (24, 8), (40, 8), (32, 4)])  # ratios 1, 4, 3, 5, 8
def test_dense_prefill_gqa_groups(device, heads):
    out, q, k, v, cu = run_dense([33, 200, 129], heads[0], heads[1], device, seed=4)
    ref = varlen_prefill_ref(q, k, v, cu, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


def _ramped(lens, device, seed, key_gain, q_gain=1.0):
    """q/k/v for `lens` with every sequence's keys scaled by key_gain(position): the running score
    maximum then rises tile after tile, past the kernel's lazy-rescale threshold (2^8) several times."""
    gen = torch.Generator(device=device).manual_seed(seed)
    t = sum(lens)
    q = (torch.randn((t, 16, 128), generator=gen, device=device) * q_gain).to(torch.bfloat16)
    k = torch.randn((t, 8, 128), generator=gen, device=device)
    pos = torch.cat([torch.arange(n, device=device) for n in lens]).float()
    k = (k * key_gain(pos)[:, None, None]).to(torch.bfloat16)
    v = rand((t, 8, 128), gen, device)
    return q, k, v


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["ramp", "large"])
def test_dense_prefill_rescales_after_the_first_tile(device, case):
    """Scores that grow along the keys (ramp) or are large everywhere (q and k ~ N(0, 9)): the
    exponent reference moves on later tiles, so O and l are rescaled mid-sequence."""
    lens = [300, 1000, 64]
    gain = (lambda pos: 1.0 + pos / 48.0) if case == "ramp" else (lambda pos: torch.full_like(pos, 3.0))
    q, k, v = _ramped(lens, device, seed=21, key_gain=gain, q_gain=1.0 if case == "ramp" else 3.0)
    cu = W.cu_seqlens(lens)
    out = torch.empty_like(q)
    _C.varlen_prefill(out, q, k, v, torch.tensor(cu, dtype=torch.int32, device=device), max(lens), SCALE)
    torch.cuda.synchronize()
    ref = varlen_prefill_ref(q, k, v, cu, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.gpu
def test_dense_prefill_fused_qkv_views(device):
    out, q, k, v, cu = run_dense([70, 150], 16, 8, device, seed=9, fused=True)
    ref = varlen_prefill_ref(q, k, v, cu, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.gpu
def test_dense_prefill_32_ragged_prompts(device):
    """32 prompts of U[64, 2048] tokens packed with cu_seqlens, 16 q / 8 kv heads."""
    lens = W.prefill_lengths(32, 64, 2048, seed=0)
    out, q, k, v, cu = run_dense(lens, 16, 8, device, seed=0)
    ref = varlen_prefill_ref(q, k, v, cu, SCALE)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL, err


@pytest.mark.gpu
def test_dense_prefill_long_prompts(device):
    """Prompts of 12,000 and 20,000 tokens (up to 625 key tiles per query tile).  The oracle
    attends a spread of rows of each prompt, its first and last tiles included, over their full
    causal prefix."""
    from oracle.attention_ref import _attend

    lens = [12000, 20000]
    out, q, k, v, cu = run_dense(lens, 16, 8, device, seed=21)
    out, q, k, v = out.float().cpu(), q.cpu(), k.cpu(), v.cpu()
    gen = torch.Generator().manual_seed(21)
    for s, n in enumerate(lens):
        a = cu[s]
        picked = torch.randint(0, n, (24,), generator=gen).tolist()
        rows = torch.tensor(sorted({0, 1, 31, 32, 63, 64, 127, 128, n // 2, n - 129, n - 64, n - 1, *picked}))
        allowed = torch.arange(n)[None, :] <= rows[:, None]
        ref = _attend(q[a + rows], k[a : a + n], v[a : a + n], SCALE, allowed)
        err = (out[a + rows] - ref).abs().max().item()
        assert err <= TOL, (n, err)


def _paged_case(device, prompt_lens, cached, bs=128, seed=0, hq=16, hkv=8, qkv=None):
    """Full prompts written to a paged cache; queries = the suffix after `cached` tokens.  `qkv`
    gives the prompts' (q, k, v) instead of seeded N(0, 1) ones."""
    gen = torch.Generator(device=device).manual_seed(seed)
    nblk = [math.ceil(n / bs) for n in prompt_lens]
    num_blocks = sum(nblk) + 3
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(seed)).tolist()
    tables = torch.zeros(len(prompt_lens), max(nblk), dtype=torch.int32)
    pos = 0
    for i, nb in enumerate(nblk):
        tables[i, :nb] = torch.tensor(perm[pos : pos + nb])
        pos += nb
    t = sum(prompt_lens)
    if qkv is None:
        q = rand((t, hq, 128), gen, device)
        k = rand((t, hkv, 128), gen, device)
        v = rand((t, hkv, 128), gen, device)
    else:
        q, k, v = qkv
    kc = torch.full((num_blocks, bs, hkv, 128), float("nan"), dtype=torch.bfloat16, device=device)
    vc = torch.full_like(kc, float("nan"))
    slots = torch.tensor([int(tables[i, p // bs]) * bs + p % bs for i, n in enumerate(prompt_lens) for p in range(n)],
                         dtype=torch.int64, device=device)
    _C.kv_cache_write(k, v, kc, vc, slots)
    cu_full = W.cu_seqlens(prompt_lens)
    sel = torch.tensor([cu_full[i] + p for i, n in enumerate(prompt_lens) for p in range(cached[i], n)],
                       device=device)
    qs = q[sel].contiguous()
    q_lens = [n - c for n, c in zip(prompt_lens, cached)]
    cu_q = W.cu_seqlens(q_lens)
    out = torch.empty_like(qs)
    _C.paged_prefill(out, qs, kc, vc, tables.to(device), torch.tensor(cu_q, dtype=torch.int32, device=device),
                     torch.tensor(prompt_lens, dtype=torch.int32, device=device), max(q_lens), SCALE)
    torch.cuda.synchronize()
    return out, qs, q, k, v, kc, vc, tables, cu_q, cu_full, sel


@pytest.mark.gpu
@pytest.mark.parametrize("bs", [128, 64, 32, 16])  # >= 32: one descriptor per tile; 16: per-row lookups
def test_paged_prefix_hit_prefill(device, bs):
    prompt_lens = [300, 129, 1000, 64, 255]
    cached = [256, 128, 384, 0, 128]
    out, qs, q, k, v, kc, vc, tables, cu_q, cu_full, sel = _paged_case(device, prompt_lens, cached, bs=bs, seed=bs)
    ref = paged_prefill_ref(qs, kc, vc, tables, cu_q, prompt_lens, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL
    # the reference's cache-hit == no-cache invariant: rows equal the dense prefill of the whole prompt
    dense = torch.empty(q.shape, dtype=torch.bfloat16, device=device)
    _C.varlen_prefill(dense, q, k, v, torch.tensor(cu_full, dtype=torch.int32, device=device), max(prompt_lens),
                      SCALE)
    torch.cuda.synchronize()
    assert (out.float() - dense[sel].float()).abs().max().item() <= TOL


@pytest.mark.gpu
def test_paged_prefill_long_cached_prefixes(device):
    """Prefix hits of 17,500 and 8,800 cached tokens (137 and 69 pages) ahead of 500 and 200 new
    query rows: against the oracle, and equal to the dense prefill rows of the whole prompts."""
    prompt_lens, cached = [18000, 9000], [17500, 8800]
    out, qs, q, k, v, kc, vc, tables, cu_q, cu_full, sel = _paged_case(device, prompt_lens, cached, seed=31)
    ref = paged_prefill_ref(qs, kc, vc, tables, cu_q, prompt_lens, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL
    dense = torch.empty(q.shape, dtype=torch.bfloat16, device=device)
    _C.varlen_prefill(dense, q, k, v, torch.tensor(cu_full, dtype=torch.int32, device=device), max(prompt_lens),
                      SCALE)
    torch.cuda.synchronize()
    assert (out.float() - dense[sel].float()).abs().max().item() <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("heads", [(40, 8), (32, 4)])
def test_paged_prefill_gqa_launch_groups(device, heads):
    """Ratios 5 and 8 run as several launches over 4, 2 and 1 query heads of every kv head."""
    prompt_lens, cached = [300, 129, 700], [256, 0, 384]
    out, qs, q, k, v, kc, vc, tables, cu_q, cu_full, sel = _paged_case(device, prompt_lens, cached, bs=64, seed=9,
                                                                       hq=heads[0], hkv=heads[1])
    ref = paged_prefill_ref(qs, kc, vc, tables, cu_q, prompt_lens, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.gpu
def test_paged_prefill_rescales_after_the_first_tile(device):
    """The paged route's softmax with keys that grow along the prompt (reference moves on later tiles)."""
    prompt_lens, cached = [700, 300], [512, 128]
    qkv = _ramped(prompt_lens, device, seed=5, key_gain=lambda pos: 1.0 + pos / 48.0)
    out, qs, q, k, v, kc, vc, tables, cu_q, cu_full, sel = _paged_case(device, prompt_lens, cached, bs=64, seed=5,
                                                                       qkv=qkv)
    ref = paged_prefill_ref(qs, kc, vc, tables, cu_q, prompt_lens, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.gpu
def test_paged_prefill_full_prompt_equals_dense(device):
    prompt_lens = [77, 513]
    out, qs, q, k, v, kc, vc, tables, cu_q, cu_full, sel = _paged_case(device, prompt_lens, [0, 0], seed=3)
    ref = varlen_prefill_ref(q, k, v, cu_full, SCALE)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL
