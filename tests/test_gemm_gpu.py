"""Skinny-M projection kernels (decode batches, M <= 128) against fp32 torch references.

The kernel accumulates in fp32 and rounds to bf16 once, so each output is within one bf16 ulp of
the fp32 product of the same bf16 operands: half an ulp is at most 2^-8 of the value, and the
additive slack covers the fp32 summation-order difference.  Weights are passed tiled
(``_C.tile``); tiled activations and outputs must give bit-identical results to row-major ones.
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
@pytest.mark.parametrize("m", [1, 7, 32, 33, 100, 128])
@pytest.mark.parametrize("nk", SHAPES, ids=[f"n{n}_k{k}" for n, k in SHAPES])
def test_linear_matches_fp32(device, m, nk):
    n, k = nk
    x, w = _operands(m, n, k, device, seed=m * 7 + n)
    y = _C.linear(x, _C.tile(w))
    ref = x.float() @ w.float().t()
    torch.cuda.synchronize()
    _assert_close_bf16(y, ref)
    # and within one ulp (2^-7 relative at most) of the library GEMM the reference model runs
    _assert_close_bf16(y, F.linear(x, w).float(), rel=2 * ULP)


def _bf16_steps(x, steps):
    """x (bf16) moved by each of `steps` representable values (bit pattern +- 1 is the next
    value up or down; which one depends on the sign, and both are covered)."""
    bits = x.view(torch.int16)
    return [(bits + d).view(torch.bfloat16) for d in steps]


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 5, 32, 77])
def test_linear_silu_mul_matches_unfused_rounding(device, m):
    """Exact check: y = bf16(bf16(silu(g)) * u) for g, u the bf16 gate and up projections.
    A different fp32 summation order may round g or u to the neighbouring bf16 value (and an
    fp32 silu may round to the neighbouring bf16), so y must equal the chain for some g', u',
    s' within one bf16 step of the fp32 reference's values."""
    inter, k = 3072, 1024
    x, w = _operands(m, 2 * inter, k, device, seed=100 + m)
    y = _C.linear_silu_mul(x, _C.tile(w))
    full = x.float() @ w.float().t()
    g = full[:, :inter].to(torch.bfloat16)
    u = full[:, inter:].to(torch.bfloat16)
    torch.cuda.synchronize()
    hit = torch.zeros_like(y, dtype=torch.bool)
    for gg in _bf16_steps(g, (-1, 0, 1)):
        for ss in _bf16_steps(F.silu(gg.float()).to(torch.bfloat16), (-1, 0, 1)):
            for uu in _bf16_steps(u, (-1, 0, 1)):
                hit |= (ss.float() * uu.float()).to(torch.bfloat16) == y
    # near g = 0 the summation-order difference spans many bf16 steps of g, but y ~ g * u / 2 is
    # then tiny: those elements are held to an absolute bound instead
    chain = (F.silu(g.float()).to(torch.bfloat16).float() * u.float()).to(torch.bfloat16).float()
    near = (y.float() - chain).abs() <= 3e-5
    bad = ~(hit | near)
    assert not bool(bad.any()), (f"{int(bad.sum())} outputs match no neighbouring rounding of the chain: "
                                 f"y={y[bad].tolist()} chain={chain[bad].tolist()} g={g[bad].tolist()} "
                                 f"u={u[bad].tolist()}")
    # and the fused launch agrees with the kernel's own unfused chain to the same rule
    two = _C.silu_mul(_C.linear(x, _C.tile(w)))
    assert ((two.float() - y.float()).abs() <= 4 * ULP * y.float().abs() + 1e-3).float().mean().item() > 0.999


@pytest.mark.gpu
def test_linear_strided_input_and_output(device):
    m, n, k = 9, 1024, 2048
    x, w = _operands(m, n, k, device, seed=3)
    xbuf = torch.zeros((m, k + 256), dtype=torch.bfloat16, device=device)
    xbuf[:, 128 : 128 + k] = x
    ybuf = torch.zeros((m, n + 64), dtype=torch.bfloat16, device=device)
    y = _C.linear(xbuf[:, 128 : 128 + k], _C.tile(w), out=ybuf[:, 32 : 32 + n])
    torch.cuda.synchronize()
    _assert_close_bf16(y, x.float() @ w.float().t())
    assert int(ybuf[:, :32].abs().sum()) == 0 and int(ybuf[:, 32 + n :].abs().sum()) == 0


@pytest.mark.gpu
def test_linear_is_deterministic(device):
    x, w = _operands(32, 4096, 1024, device, seed=8)
    wt = _C.tile(w)
    a = _C.linear(x, wt)
    b = _C.linear(x, wt)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_linear_rejects_more_than_128_rows(device):
    x, w = _operands(129, 1024, 1024, device, seed=9)
    with pytest.raises(ValueError):
        _C.linear(x, _C.tile(w))


@pytest.mark.gpu
def test_linear_rejects_a_row_major_weight(device):
    x, w = _operands(4, 1024, 1024, device, seed=9)
    with pytest.raises(ValueError):
        _C.linear(x, w)


def _tile_ssq(x):
    """Per-32-column sums of squares of a bf16 [M, K] tensor, fp32 [M, K/32]."""
    m, k = x.shape
    return (x.float() ** 2).view(m, k // 32, 32).sum(-1)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 13, 32, 48, 100])
@pytest.mark.parametrize("nk", [(4096, 1024), (151936, 1024), (1024, 2048)], ids=["qkv", "lm_head", "k2048"])
def test_norm_prologue_matches_add_rms_norm_then_linear(device, m, nk):
    """Above 32 rows the kernel takes 64-row slabs for k <= 1024 (one slab at 48 rows, two at 100)
    and 32-row slabs for a larger k (k2048)."""
    n, k = nk
    x, w = _operands(m, n, k, device, seed=31 + m)
    gen = torch.Generator(device=device).manual_seed(5)
    nw = (1.0 + 0.02 * torch.randn(k, generator=gen, device=device)).to(torch.bfloat16)
    ssq = _tile_ssq(x).contiguous()
    wt = _C.tile(w)
    y = _C.skinny_linear(x, wt, x_ssq=ssq, norm_weight=nw, eps=1e-6)
    # the unfused chain: the standalone RMSNorm kernel, then the plain projection
    a = torch.empty_like(x)
    _C.add_rms_norm(None, x.clone(), nw, a, 1e-6)
    y2 = _C.linear(a, wt)
    # fp32 emulation of the prologue's rounding
    rstd = torch.rsqrt(ssq.sum(-1, keepdim=True) / k + 1e-6)
    a_ref = ((x.float() * rstd) * nw.float()).to(torch.bfloat16)
    ref = a_ref.float() @ w.float().t()
    torch.cuda.synchronize()
    # an operand element may round the other way (different fp32 order of the sum of squares):
    # allow one ulp of the product's scale on top of the output rounding
    scale = ref.abs().amax(dim=1, keepdim=True)
    assert ((y.float() - ref).abs() <= 2 * ULP * ref.abs() + 0.02 * ULP * scale).all()
    assert ((y.float() - y2.float()).abs() <= 2 * ULP * ref.abs() + 0.02 * ULP * scale).all()


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 32, 100])
@pytest.mark.parametrize("nk", [(1024, 2048), (1024, 3072), (1024, 1024), (2048, 4096), (4096, 1024)],
                         ids=["o_proj", "down_proj", "split4_k1024", "split2_k4096", "unsplit_n4096"])
def test_residual_epilogue(device, m, nk):
    """The residual epilogue over the K splits the plan picks (4 for n = 1024, 2 for n = 2048, none
    for n = 4096): fp32-reference bound, the sums of squares of what was written, and agreement
    with the standalone residual-add kernel."""
    n, k = nk
    x, w = _operands(m, n, k, device, seed=71 + k + m)
    gen = torch.Generator(device=device).manual_seed(6)
    r0 = torch.randn((m, n), generator=gen, device=device).to(torch.bfloat16)
    r = r0.clone()
    ssq = torch.full((m, n // 32), -1.0, device=device)
    _C.skinny_linear(x, _C.tile(w), r, epilogue=_C.EPI_RESID, y_ssq=ssq)
    d_ref = (x.float() @ w.float().t())
    torch.cuda.synchronize()
    d = d_ref.to(torch.bfloat16).float()
    r_ref = r0.float() + d
    bound = 2 * ULP * (d.abs() + r_ref.abs()) + 1e-6
    assert ((r.float() - r_ref).abs() <= bound).all()
    # the sums of squares are those of the residual the kernel wrote
    assert torch.allclose(ssq, _tile_ssq(r), rtol=1e-5, atol=1e-6)
    # and the same as the standalone residual-add kernel applied to the projection
    r2 = r0.clone()
    _C.add_rms_norm(_C.linear(x, _C.tile(w)), r2, torch.ones(n, dtype=torch.bfloat16, device=device),
                    torch.empty_like(r2), 1e-6)
    torch.cuda.synchronize()
    assert ((r.float() - r2.float()).abs() <= bound).all()


@pytest.mark.gpu
def test_embed_rows_and_sums_of_squares(device):
    gen = torch.Generator(device=device).manual_seed(7)
    table = torch.randn((5000, 1024), generator=gen, device=device).to(torch.bfloat16)
    ids = torch.tensor([0, 4999, 17, -1, 5000, 17], dtype=torch.int64, device=device)
    ssq = torch.full((6, 32), -1.0, device=device)
    out = _C.embed_rows(ids, table, ssq=ssq)
    torch.cuda.synchronize()
    assert torch.equal(out[[0, 1, 2, 5]], table[[0, 4999, 17, 17]])
    assert int(out[[3, 4]].abs().sum()) == 0  # ids outside the vocab give zero rows
    assert torch.allclose(ssq, _tile_ssq(out), rtol=1e-5, atol=1e-6)


@pytest.mark.gpu
def test_split_k_is_deterministic_and_leaves_workspace_zero(device):
    ws = torch.zeros(max(_C.skinny_linear_workspace_size(1024, k, e) for k in (2048, 3072) for e in (0, 2))
                     + max(_C.skinny_linear_workspace_size(3072, 1024, 1), 0), dtype=torch.uint8, device=device)
    assert ws.numel() > 0
    outs = []
    for rep in range(3):
        for k in (2048, 3072):
            x, w = _operands(100, 1024, k, device, seed=k)
            m = 100 if rep == 1 else 32  # rows are independent: the first 32 of 100 equal a 32-row call
            outs.append((rep, k, _C.linear(x[:m], _C.tile(w), workspace=ws)[:32]))
    torch.cuda.synchronize()
    by_k = {}
    for rep, k, y in outs:
        by_k.setdefault(k, []).append(y)
    for ys in by_k.values():
        assert all(torch.equal(ys[0], y) for y in ys[1:])
    assert int(ws[:4096 * 4].view(torch.int32).abs().sum()) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("m", [32, 100])
def test_graph_replays_equal_eager(device, m):
    """A captured decode-style chain (norm prologue, SiLU, residual) replays to the eager result."""
    h, inter = 1024, 3072
    gen = torch.Generator(device=device).manual_seed(8)
    w_gu = _C.tile((torch.randn((2 * inter, h), generator=gen, device=device) * 0.02).to(torch.bfloat16))
    w_dn = _C.tile((torch.randn((h, inter), generator=gen, device=device) * 0.02).to(torch.bfloat16))
    nw = (1.0 + 0.02 * torch.randn(h, generator=gen, device=device)).to(torch.bfloat16)
    ws = torch.zeros(max(_C.skinny_linear_workspace_size(inter, h, 1), _C.skinny_linear_workspace_size(h, inter, 2)),
                     dtype=torch.uint8, device=device)
    r = _C.tiled_empty(m, h, device)  # the residual stream and the SiLU output tiled, as the model keeps them
    ssq = torch.empty((m, h // 32), device=device)
    act = _C.tiled_empty(m, inter, device)

    def chain():
        _C.skinny_linear(r, w_gu, act, epilogue=_C.EPI_SILU, x_ssq=ssq, norm_weight=nw, workspace=ws, m=m,
                         y_tiled=True)
        _C.skinny_linear(act, w_dn, r, epilogue=_C.EPI_RESID, y_ssq=ssq, workspace=ws, m=m, y_tiled=True)

    def reset(seed):
        g = torch.Generator(device=device).manual_seed(seed)
        x = torch.randn((m, h), generator=g, device=device).to(torch.bfloat16)
        r.copy_(_C.tile(x))
        ssq.copy_(_tile_ssq(x))

    reset(1)
    chain()  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    for seed in (2, 3, 4):
        reset(seed)
        graph.replay()
        torch.cuda.synchronize()
        got_r, got_ssq = r.clone(), ssq.clone()
        reset(seed)
        chain()
        torch.cuda.synchronize()
        assert torch.equal(got_r, r) and torch.equal(got_ssq, ssq)


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 13, 17, 32, 49, 100, 128])
@pytest.mark.parametrize("epi", [_C.EPI_STORE, _C.EPI_SILU, _C.EPI_RESID], ids=["store", "silu", "resid"])
def test_tiled_activations_equal_row_major(device, m, epi):
    """The same projection with x and y tiled gives the row-major results bit for bit (the same
    fragments in the same order); padding rows of a tiled x -- here NaN -- reach only dropped
    outputs, and padding rows of a tiled y are never written."""
    n, k = {_C.EPI_STORE: (4096, 1024), _C.EPI_SILU: (3072, 1024), _C.EPI_RESID: (1024, 3072)}[epi]
    wrows = 2 * n if epi == _C.EPI_SILU else n
    x, w = _operands(m, wrows, k, device, seed=200 + m + epi)
    wt = _C.tile(w)
    rows = 16 * -(-m // 16)
    norm = epi != _C.EPI_RESID
    gen = torch.Generator(device=device).manual_seed(11)
    nw = (1.0 + 0.02 * torch.randn(k, generator=gen, device=device)).to(torch.bfloat16) if norm else None
    x_ssq = _tile_ssq(x).contiguous() if norm else None
    ws = torch.zeros(max(_C.skinny_linear_workspace_size(n, k, epi), 16), dtype=torch.uint8, device=device)
    x_pad = torch.full((rows, k), float("nan"), dtype=torch.bfloat16, device=device)
    x_pad[:m] = x
    xt = _C.tile(x_pad)
    y_pad = torch.full((rows, n), 7.0, dtype=torch.bfloat16, device=device)  # sentinel rows past m
    if epi == _C.EPI_RESID:
        r0 = torch.randn((m, n), generator=gen, device=device).to(torch.bfloat16)
        y_rm, ssq_rm = r0.clone(), torch.zeros((m, n // 32), device=device)
        _C.skinny_linear(x, wt, y_rm, epilogue=epi, y_ssq=ssq_rm, workspace=ws)
        y_pad[:m] = r0
        yt = _C.tile(y_pad)
        ssq_t = torch.zeros((m, n // 32), device=device)
        _C.skinny_linear(xt, wt, yt, epilogue=epi, y_ssq=ssq_t, workspace=ws, m=m, y_tiled=True)
        torch.cuda.synchronize()
        assert torch.equal(ssq_t, ssq_rm)
    else:
        y_rm = _C.skinny_linear(x, wt, epilogue=epi, x_ssq=x_ssq, norm_weight=nw, workspace=ws)
        yt = _C.tile(y_pad)
        _C.skinny_linear(xt, wt, yt, epilogue=epi, x_ssq=x_ssq, norm_weight=nw, workspace=ws, m=m, y_tiled=True)
        torch.cuda.synchronize()
    got = _C.untile(yt)
    assert torch.equal(got[:m], y_rm)
    assert bool((got[m:] == 7.0).all())


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 6, 16, 27])
def test_embed_rows_tiled(device, rows):
    gen = torch.Generator(device=device).manual_seed(12)
    table = torch.randn((3000, 1024), generator=gen, device=device).to(torch.bfloat16)
    ids = torch.randint(-2, 3002, (rows,), generator=gen, device=device)
    ssq_rm, ssq_t = torch.zeros((rows, 32), device=device), torch.zeros((rows, 32), device=device)
    ref = _C.embed_rows(ids, table, ssq=ssq_rm)
    out = _C.tile(torch.full((16 * -(-rows // 16), 1024), 7.0, dtype=torch.bfloat16, device=device))
    _C.embed_rows(ids, table, out=out, ssq=ssq_t, out_tiled=True)
    torch.cuda.synchronize()
    got = _C.untile(out)
    assert torch.equal(got[:rows], ref) and torch.equal(ssq_t, ssq_rm)
    assert bool((got[rows:] == 7.0).all())


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(6))
def test_random_rows_and_epilogues(device, seed):
    """Seeded random row counts around the slab boundaries (16, 32, 64, 65, 112, 128 rows), each
    epilogue, with and without the norm prologue: every row equals the same projection of that row
    alone (rows are independent; a one-row call takes the smallest configuration), bit for bit."""
    import random
    rng = random.Random(1000 + seed)
    shapes = {_C.EPI_STORE: [(4096, 1024), (1024, 2048)], _C.EPI_SILU: [(3072, 1024)],
              _C.EPI_RESID: [(1024, 2048), (1024, 3072)]}
    for _ in range(3):
        epi = rng.choice(list(shapes))
        n, k = rng.choice(shapes[epi])
        m = rng.choice([rng.randint(1, 128), rng.choice([16, 17, 32, 33, 63, 64, 65, 96, 112, 113, 127, 128])])
        norm = epi != _C.EPI_RESID and rng.random() < 0.5
        wrows = 2 * n if epi == _C.EPI_SILU else n
        x, w = _operands(m, wrows, k, device, seed=seed * 101 + m)
        wt = _C.tile(w)
        gen = torch.Generator(device=device).manual_seed(seed)
        nw = (1.0 + 0.02 * torch.randn(k, generator=gen, device=device)).to(torch.bfloat16) if norm else None
        ssq = _tile_ssq(x).contiguous() if norm else None
        ws = torch.zeros(max(_C.skinny_linear_workspace_size(n, k, epi), 16), dtype=torch.uint8, device=device)
        if epi == _C.EPI_RESID:
            r0 = torch.randn((m, n), generator=gen, device=device).to(torch.bfloat16)
            y = r0.clone()
            _C.skinny_linear(x, wt, y, epilogue=epi, y_ssq=torch.zeros((m, n // 32), device=device), workspace=ws)
        else:
            y = _C.skinny_linear(x, wt, epilogue=epi, x_ssq=ssq, norm_weight=nw, workspace=ws)
        for row in sorted({0, m // 2, m - 1}):
            sl = slice(row, row + 1)
            if epi == _C.EPI_RESID:
                y1 = r0[sl].clone()
                _C.skinny_linear(x[sl], wt, y1, epilogue=epi, y_ssq=torch.zeros((1, n // 32), device=device),
                                 workspace=ws)
            else:
                y1 = _C.skinny_linear(x[sl], wt, epilogue=epi, x_ssq=None if ssq is None else ssq[sl].contiguous(),
                                      norm_weight=nw, workspace=ws)
            torch.cuda.synchronize()
            assert torch.equal(y[sl], y1), (f"epilogue {epi} norm {norm} m {m} n {n} k {k} row {row}: "
                                            f"max diff {(y[sl].float() - y1.float()).abs().max().item():.3g}")
