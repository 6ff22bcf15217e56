"""Skinny-M projection kernels (decode batches, M <= 32) against fp32 torch references.

The kernel accumulates in fp32 and rounds to bf16 once, so each output is within one bf16 ulp of
the fp32 product of the same bf16 operands: half an ulp is at most 2^-8 of the value, and the
additive slack covers the fp32 summation-order difference.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from nano_vllm_ascend_amd import _C

ULP = 2.0 ** -8

# (n, k) of the Qwen3-0.6B decode projections: qkv, o, down, LM head
SHAPES = [(4096, 1024), (1024, 2048), (1024, 3072), (151936, 1024)]


def _operands(m, n, k, device, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn((m, k), generator=gen, device=device).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=gen, device=device) * 0.02).to(torch.bfloat16)
    return x, w


def _assert_close_bf16(y, ref, rel=ULP, slack=1e-5):
    err = (y.float() - ref).abs()
    bound = rel * ref.abs() + slack
    bad = (err > bound).sum().item()
    assert bad == 0, f"{bad} elements beyond one bf16 ulp; worst {err.max().item():.3g}"


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 7, 32])
@pytest.mark.parametrize("nk", SHAPES, ids=[f"n{n}_k{k}" for n, k in SHAPES])
def test_linear_matches_fp32(device, m, nk):
    n, k = nk
    x, w = _operands(m, n, k, device, seed=m * 7 + n)
    y = _C.linear(x, w)
    ref = x.float() @ w.float().t()
    torch.cuda.synchronize()
    _assert_close_bf16(y, ref)
    # and within one ulp (2^-7 relative at most) of the library GEMM the reference model runs
    _assert_close_bf16(y, F.linear(x, w).float(), rel=2 * ULP)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 5, 32])
def test_linear_silu_mul_matches_unfused_rounding(device, m):
    inter, k = 3072, 1024
    x, w = _operands(m, 2 * inter, k, device, seed=100 + m)
    y = _C.linear_silu_mul(x, w)
    full = x.float() @ w.float().t()
    g = full[:, :inter].to(torch.bfloat16).float()
    u = full[:, inter:].to(torch.bfloat16).float()
    ref = (F.silu(g).to(torch.bfloat16).float() * u)
    torch.cuda.synchronize()
    # g and u may each sit one rounding away from the kernel's: allow two ulps of the product
    err = (y.float() - ref).abs()
    bound = 2 * ULP * ref.abs() + 1e-4
    assert int((err > bound).sum()) == 0, f"worst {err.max().item():.3g}"
    # and the fused launch equals the kernel's own unfused chain up to those roundings
    two = _C.silu_mul(_C.linear(x, w))
    assert (two.float() - y.float()).abs().max().item() <= 2 * ULP * ref.abs().max().item() + 1e-4


@pytest.mark.gpu
def test_linear_strided_input_and_output(device):
    m, n, k = 9, 1024, 2048
    x, w = _operands(m, n, k, device, seed=3)
    xbuf = torch.zeros((m, k + 256), dtype=torch.bfloat16, device=device)
    xbuf[:, 128 : 128 + k] = x
    ybuf = torch.zeros((m, n + 64), dtype=torch.bfloat16, device=device)
    y = _C.linear(xbuf[:, 128 : 128 + k], w, out=ybuf[:, 32 : 32 + n])
    torch.cuda.synchronize()
    _assert_close_bf16(y, x.float() @ w.float().t())
    assert int(ybuf[:, :32].abs().sum()) == 0 and int(ybuf[:, 32 + n :].abs().sum()) == 0


@pytest.mark.gpu
def test_linear_is_deterministic(device):
    x, w = _operands(32, 4096, 1024, device, seed=8)
    a = _C.linear(x, w)
    b = _C.linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_linear_rejects_more_than_32_rows(device):
    x, w = _operands(33, 1024, 1024, device, seed=9)
    with pytest.raises(ValueError):
        _C.linear(x, w)
