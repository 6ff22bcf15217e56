"""Parity of the fused elementwise HIP kernels (add+RMSNorm, SiLU*mul, argmax) with torch references."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from nano_vllm_ascend_amd import _C


def _bf(shape, gen, device, scale=1.0):
    return (torch.randn(shape, generator=gen, device=device) * scale).to(torch.bfloat16)


@pytest.mark.gpu
# 2560 (Qwen3-4B), 5120 (-14B / -32B), 8200 and 8: the any-width kernel
@pytest.mark.parametrize("rows,hidden", [(1, 1024), (33, 1024), (5, 2048), (7, 4096), (9, 2560), (6, 5120),
                                         (3, 8200), (70, 8)])
def test_add_rms_norm_matches_reference_rounding(device, rows, hidden):
    g = torch.Generator(device=device).manual_seed(rows)
    res = _bf((rows, hidden), g, device)
    delta = _bf((rows, hidden), g, device)
    w = (1 + 0.1 * torch.randn(hidden, generator=g, device=device)).to(torch.bfloat16)
    # reference: bf16 residual add, then fp32 RMSNorm with one rounding (nv/models/qwen3.py:138-150)
    new_res = (res.float() + delta.float()).to(torch.bfloat16)
    x = new_res.float()
    ref = (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()).to(torch.bfloat16)
    out = torch.empty_like(res)
    _C.add_rms_norm(delta, res, w, out, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(res, new_res)
    # the fp32 sum of squares is accumulated in a different order than torch's, so an
    # element may round to the neighbouring bf16 value: at most one ulp (relative 2^-7)
    diff = (out.float() - ref.float()).abs()
    assert bool((diff <= ref.float().abs() * 2.0 ** -7 + 1e-6).all())
    assert (diff == 0).float().mean().item() > 0.99
    out2 = torch.empty_like(res)
    _C.add_rms_norm(None, res, w, out2, 1e-6)  # plain norm leaves the residual alone
    torch.cuda.synchronize()
    assert torch.equal(res, new_res)
    assert bool(((out2.float() - ref.float()).abs() <= ref.float().abs() * 2.0 ** -7 + 1e-6).all())


@pytest.mark.gpu
def test_silu_mul_matches_torch(device):
    g = torch.Generator(device=device).manual_seed(0)
    gu = _bf((37, 2 * 3072), g, device, 3.0)
    ref = F.silu(gu[:, :3072]) * gu[:, 3072:]
    out = _C.silu_mul(gu)
    torch.cuda.synchronize()
    diff = (out.float() - ref.float()).abs()
    assert diff.max().item() <= 0.05 and (diff == 0).float().mean().item() > 0.99


@pytest.mark.gpu
def test_argmax_rows_first_index_on_ties(device):
    g = torch.Generator(device=device).manual_seed(1)
    logits = _bf((32, 151936), g, device)
    logits[3, 100] = 9.0
    logits[3, 50000] = 9.0  # tie: the first index wins
    logits[7, 151935] = 9.5  # the last (unvectorised tail) element
    logits[9].fill_(1.0)  # all equal: index 0
    out = _C.argmax_rows(logits)
    torch.cuda.synchronize()
    assert out.tolist() == logits.float().argmax(dim=-1).tolist()
    assert out[3].item() == 100 and out[7].item() == 151935 and out[9].item() == 0


@pytest.mark.gpu
def test_argmax_rows_ragged_vocab_and_ties_within_a_thread(device):
    """A vocab that is not a multiple of 8 (scalar tail), strided rows, and ties that one thread
    meets in different load slots of a step or in different steps (the first index wins)."""
    g = torch.Generator(device=device).manual_seed(2)
    vocab = 151939
    buf = _bf((6, 151944), g, device)
    logits = buf[:, :vocab]
    logits[0, 8] = 7.0
    logits[0, 8 + 8192] = 7.0        # same thread, next load slot
    logits[1, 24] = 7.0
    logits[1, 24 + 4 * 8192] = 7.0   # same thread, next step
    logits[2, vocab - 1] = 7.0       # scalar tail
    logits[3, vocab - 3] = 7.0
    logits[3, 5] = 7.0               # tie between the vector body and the tail
    buf[4, vocab:] = 50.0            # padding past vocab is never read as a logit
    logits[5].fill_(-1.0)
    out = _C.argmax_rows(logits)
    torch.cuda.synchronize()
    assert out.tolist() == [8, 24, vocab - 1, 5, logits[4].float().argmax().item(), 0]
