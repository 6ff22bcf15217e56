"""Pins for the CPU oracle: library routines, brute force, invariants and planted mistakes (CPU only).

Retyping the oracle's formula would pin nothing, so every check compares it
with an independent computation: torch SDPA, HF transformers' Qwen3 layers,
explicit loops on tiny inputs, or a mathematical invariant.  Two tests plant
a plausible mistake in a copy of the oracle and show that the checks catch it.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention_ref as A
from oracle.qwen3_ref import Qwen3Ref, load_into_hf

torch.manual_seed(0)


def _paged(ctx_lens, hkv=2, d=16, bs=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    nblk = [math.ceil(c / bs) for c in ctx_lens]
    nb = sum(nblk) + 2
    perm = torch.randperm(nb, generator=g)
    bt = torch.zeros(len(ctx_lens), max(nblk), dtype=torch.int32)
    p = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[p : p + n]
        p += n
    kc = torch.randn(nb, bs, hkv, d, generator=g)
    vc = torch.randn(nb, bs, hkv, d, generator=g)
    return kc, vc, bt


def test_paged_decode_matches_sdpa_on_gathered_kv():
    ctx = [1, 5, 9, 16]
    kc, vc, bt = _paged(ctx)
    q = torch.randn(4, 4, 16)
    out = A.paged_decode_ref(q, kc, vc, bt, torch.tensor(ctx), 0.25)
    for i, c in enumerate(ctx):
        k = torch.cat([kc[int(bt[i, j // 4]), j % 4] [None] for j in range(c)])  # [c, Hkv, D], row by row
        v = torch.cat([vc[int(bt[i, j // 4]), j % 4][None] for j in range(c)])
        ref = F.scaled_dot_product_attention(q[i][:, None], k.transpose(0, 1), v.transpose(0, 1), scale=0.25,
                                             enable_gqa=True)[:, 0]
        assert torch.allclose(out[i], ref, atol=1e-5)


def test_paged_decode_brute_force_tiny():
    ctx = [3, 6]
    kc, vc, bt = _paged(ctx, hkv=1, d=4, bs=2, seed=1)
    q = torch.randn(2, 2, 4)
    out = A.paged_decode_ref(q, kc, vc, bt, torch.tensor(ctx), 0.5)
    for i, c in enumerate(ctx):
        for h in range(2):
            scores, rows = [], []
            for j in range(c):
                blk, off = int(bt[i, j // 2]), j % 2
                scores.append(sum(float(q[i, h, x]) * float(kc[blk, off, 0, x]) for x in range(4)) * 0.5)
                rows.append(vc[blk, off, 0])
            m = max(scores)
            e = [math.exp(s - m) for s in scores]
            ref = sum(w * r for w, r in zip(e, rows)) / sum(e)
            assert torch.allclose(out[i, h], ref, atol=1e-5)


def test_decode_equals_last_row_of_causal_prefill():
    n, hq, hkv, d = 11, 4, 2, 16
    q, k, v = torch.randn(n, hq, d), torch.randn(n, hkv, d), torch.randn(n, hkv, d)
    dense = A.varlen_prefill_ref(q, k, v, [0, n], 0.3)
    kc = k.view(n, 1, hkv, d)  # one-token pages, identity table
    vc = v.view(n, 1, hkv, d)
    bt = torch.arange(n, dtype=torch.int32)[None]
    dec = A.paged_decode_ref(q[-1:], kc, vc, bt, torch.tensor([n]), 0.3)
    assert torch.allclose(dec[0], dense[-1], atol=1e-5)


def test_varlen_prefill_matches_sdpa_causal_gqa():
    lens = [1, 7, 19]
    t = sum(lens)
    q, k, v = torch.randn(t, 8, 32), torch.randn(t, 4, 32), torch.randn(t, 4, 32)
    cu = [0, 1, 8, 27]
    out = A.varlen_prefill_ref(q, k, v, cu, 32 ** -0.5)
    for a, b in zip(cu[:-1], cu[1:]):
        ref = F.scaled_dot_product_attention(q[a:b].transpose(0, 1), k[a:b].transpose(0, 1), v[a:b].transpose(0, 1),
                                             is_causal=True, enable_gqa=True).transpose(0, 1)
        assert torch.allclose(out[a:b], ref, atol=1e-5)


def test_varlen_prefill_matches_hf_eager_attention():
    from transformers.models.qwen3.modeling_qwen3 import eager_attention_forward

    n = 13
    q, k, v = torch.randn(n, 4, 16), torch.randn(n, 2, 16), torch.randn(n, 2, 16)
    out = A.varlen_prefill_ref(q, k, v, [0, n], 0.25)
    mask = torch.full((n, n), float("-inf")).triu(1)[None, None]

    class M(torch.nn.Module):
        num_key_value_groups = 2
        training = False

    ref, _ = eager_attention_forward(M(), q.transpose(0, 1)[None], k.transpose(0, 1)[None], v.transpose(0, 1)[None],
                                     mask, scaling=0.25)
    assert torch.allclose(out, ref[0], atol=1e-5)


def test_paged_prefill_rows_equal_dense_rows_of_full_prompt():
    lens, cached = [9, 14], [4, 8]
    hkv, d, bs = 2, 16, 4
    kc, vc, bt = _paged(lens, hkv, d, bs, seed=2)
    t = sum(lens)
    q, k, v = torch.randn(t, 4, d), torch.randn(t, hkv, d), torch.randn(t, hkv, d)
    cu = [0, 9, 23]
    for i, n in enumerate(lens):  # place the prompt's K/V in its pages
        for p in range(n):
            kc[int(bt[i, p // bs]), p % bs] = k[cu[i] + p]
            vc[int(bt[i, p // bs]), p % bs] = v[cu[i] + p]
    dense = A.varlen_prefill_ref(q, k, v, cu, 0.25)
    sel = [cu[i] + p for i, n in enumerate(lens) for p in range(cached[i], n)]
    qlens = [n - c for n, c in zip(lens, cached)]
    paged = A.paged_prefill_ref(q[sel], kc, vc, bt, [0, qlens[0], sum(qlens)], lens, 0.25)
    assert torch.allclose(paged, dense[sel], atol=1e-5)


def test_kv_write_closed_form_and_untouched_slots():
    kc = torch.randn(4, 4, 2, 8)
    vc = torch.randn(4, 4, 2, 8)
    k, v = torch.randn(3, 2, 8), torch.randn(3, 2, 8)
    slots = torch.tensor([5, -1, 14])
    nk, nv = A.kv_write_ref(k, v, kc, vc, slots)
    assert torch.equal(nk.view(16, 2, 8)[5], k[0]) and torch.equal(nk.view(16, 2, 8)[14], k[2])
    keep = [i for i in range(16) if i not in (5, 14)]
    assert torch.equal(nk.view(16, 2, 8)[keep], kc.view(16, 2, 8)[keep])
    assert torch.equal(nv.view(16, 2, 8)[keep], vc.view(16, 2, 8)[keep])


def test_rope_table_matches_hf_and_invariants():
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    cos, sin = A.rope_cos_sin_table(128, 4096, 1e6)
    cfg = Qwen3Config(head_dim=128, rope_theta=1e6, max_position_embeddings=4096, hidden_size=1024,
                      num_attention_heads=8)
    hf = Qwen3RotaryEmbedding(cfg)
    pos = torch.tensor([[0, 1, 7, 100, 4095]])
    hc, hs = hf(torch.zeros(1, 5, 128), pos)
    assert torch.allclose(cos[pos[0]], hc[0], atol=1e-5) and torch.allclose(sin[pos[0]], hs[0], atol=1e-5)
    x = torch.randn(3, 2, 128).to(torch.bfloat16)
    y = A.rope_ref(x, cos[[0, 0, 0]], sin[[0, 0, 0]])
    assert torch.equal(y, x)  # position 0 is the identity
    y = A.rope_ref(x, cos[[5, 900, 4000]], sin[[5, 900, 4000]]).float()
    xf = x.float()
    pair = lambda z: z[..., :64] ** 2 + z[..., 64:] ** 2  # noqa: E731
    assert torch.allclose(pair(y), pair(xf), rtol=3e-2, atol=3e-2)  # rotation keeps each (d, d+64) norm


def test_qk_norm_rope_matches_hf_layers():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb

    t = 6
    q = torch.randn(t, 16, 128).to(torch.bfloat16)
    k = torch.randn(t, 8, 128).to(torch.bfloat16)
    qw = (1 + 0.02 * torch.randn(128)).to(torch.bfloat16)
    kw = (1 + 0.02 * torch.randn(128)).to(torch.bfloat16)
    pos = torch.tensor([0, 3, 17, 255, 1000, 2303])
    oq, ok = A.qk_norm_rope_ref(q, k, qw, kw, pos, 1e6, 1e-6, 4096)
    nq, nk = Qwen3RMSNorm(128, 1e-6), Qwen3RMSNorm(128, 1e-6)
    nq.weight.data, nk.weight.data = qw.clone(), kw.clone()
    cos, sin = A.rope_cos_sin_table(128, 4096, 1e6)
    c, s = cos[pos].to(torch.bfloat16), sin[pos].to(torch.bfloat16)
    hq, hk = apply_rotary_pos_emb(nq(q).transpose(0, 1)[None], nk(k).transpose(0, 1)[None], c[None], s[None])
    for got, ref in ((oq, hq[0].transpose(0, 1)), (ok, hk[0].transpose(0, 1))):
        # HF rounds before the weight multiply and inside RoPE; one or two bf16 ulps apart
        assert (got.float() - ref.float()).abs().max().item() <= 0.07
        assert (got.float() - ref.float()).abs().mean().item() <= 2e-3
    unit = A.rms_norm_head_ref(q, torch.ones(128), 1e-6).float()
    assert torch.allclose(unit.pow(2).mean(-1), torch.ones(t, 16), atol=2e-2)


def _tiny_config():
    from nano_vllm_ascend_amd.config import Qwen3Config as Cfg

    return Cfg(vocab_size=503, hidden_size=256, intermediate_size=384, num_hidden_layers=2, num_attention_heads=4,
               num_key_value_heads=2, head_dim=64, max_position_embeddings=512)


def _tiny_state(cfg, seed=0):
    from nano_vllm_ascend_amd.qwen3 import Qwen3ForCausalLM

    m = Qwen3ForCausalLM(cfg)
    m.init_random(seed, std=0.05)
    with torch.no_grad():  # non-trivial norm weights
        for name, p in m.named_parameters():
            if name.endswith("norm.weight"):
                p.add_(0.1 * torch.randn(p.shape))
    return {k: v.detach().clone() for k, v in m.state_dict().items()}


def test_qwen3_oracle_fp32_matches_hf_model():
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = _tiny_config()
    state = _tiny_state(cfg)
    hf_cfg = Qwen3Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                         intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
                         num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
                         head_dim=cfg.head_dim, rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_norm_eps,
                         max_position_embeddings=cfg.max_position_embeddings, tie_word_embeddings=True,
                         attn_implementation="eager")
    hf = Qwen3ForCausalLM(hf_cfg).eval()
    load_into_hf(state, hf, cfg)
    ref = Qwen3Ref(state, cfg, round_bf16=False, max_positions=512)
    toks = [5, 77, 300, 12, 9, 480, 1]
    logits = ref.forward(toks[:5])
    logits2 = ref.forward(toks[5:])  # incremental decode through the oracle's cache
    with torch.no_grad():
        hf_logits = hf(torch.tensor([toks])).logits[0]
    assert torch.allclose(logits, hf_logits[4], atol=1e-4)
    assert torch.allclose(logits2, hf_logits[-1], atol=1e-4)


def test_qwen3_oracle_batched_and_fp64_modes_agree_with_single_sequence_fp32():
    """forward_batch runs each sequence on its own cache: row i equals the single-sequence forward of
    sequence i (fp32, to summation order); fp64 arithmetic agrees with fp32 to fp32 rounding."""
    cfg = _tiny_config()
    state = _tiny_state(cfg, seed=2)
    prompts = [[5, 77, 300, 12], [9, 480, 1, 33], [7, 7, 7, 7]]
    nxt = [[40], [41], [42]]
    single = []
    for p, n in zip(prompts, nxt):
        ref = Qwen3Ref(state, cfg, round_bf16=False, max_positions=64)
        single.append((ref.forward(p), ref.forward(n)))
    for dtype in (torch.float32, torch.float64):
        batch = Qwen3Ref(state, cfg, round_bf16=False, max_positions=64, dtype=dtype)
        batch.reset(len(prompts))
        first, second = batch.forward_batch(prompts), batch.forward_batch(nxt)
        for i, (a, b) in enumerate(single):
            assert torch.allclose(first[i], a, atol=2e-5) and torch.allclose(second[i], b, atol=2e-5), (dtype, i)
    # the sequences must not see each other: a different second prompt leaves row 0 unchanged
    other = Qwen3Ref(state, cfg, round_bf16=False, max_positions=64)
    other.reset(2)
    assert torch.allclose(other.forward_batch([prompts[0], prompts[1][::-1]])[0], single[0][0], atol=2e-5)
    with pytest.raises(ValueError):
        other.forward_batch([[1, 2], [3]])


def test_qwen3_oracle_bf16_logits_and_rounded_probabilities():
    """bf16 mode returns logits the reference's bf16 LM head can produce (exact bf16 values); rounding
    softmax probabilities to bf16 changes nothing where every probability is 1 (one key: the first
    token) and changes the logits by rounding only elsewhere."""
    cfg = _tiny_config()
    state = _tiny_state(cfg, seed=3)
    plain = Qwen3Ref(state, cfg, round_bf16=True, max_positions=64)
    probs = Qwen3Ref(state, cfg, round_bf16=True, max_positions=64, round_probs=True)
    a, b = plain.forward([11]), probs.forward([11])
    assert torch.equal(a, a.to(torch.bfloat16).float())
    assert torch.equal(a, b)  # softmax over one key is exactly 1.0 in both
    a, b = plain.forward([12, 13, 14]), probs.forward([12, 13, 14])
    assert 0 < (a - b).abs().max().item() < 0.1


# --- planted mistakes: plausible bugs that the pins above must catch ---
def test_planted_gqa_mapping_error_is_caught(monkeypatch):
    def wrong_attend(q, k, v, scale, allowed):  # kv head h % Hkv instead of h // group
        hq, hkv = q.shape[1], k.shape[1]
        idx = torch.arange(hq) % hkv
        s = torch.einsum("qhd,khd->hqk", q.float(), k.float()[:, idx]) * scale
        if allowed is not None:
            s = s.masked_fill(~allowed.unsqueeze(0), float("-inf"))
        return torch.einsum("hqk,khd->qhd", torch.softmax(s, -1), v.float()[:, idx])

    monkeypatch.setattr(A, "_attend", wrong_attend)
    with pytest.raises(AssertionError):
        test_varlen_prefill_matches_sdpa_causal_gqa()


def test_planted_rotate_half_sign_error_is_caught(monkeypatch):
    def wrong_rope(x, cos, sin):
        half = x.shape[-1] // 2
        xf = x.float()
        c = cos.to(torch.bfloat16).float().unsqueeze(1)
        s = sin.to(torch.bfloat16).float().unsqueeze(1)
        rot = torch.cat((xf[..., half:], -xf[..., :half]), dim=-1)  # sign flipped
        return (xf * c + rot * s).to(torch.bfloat16)

    monkeypatch.setattr(A, "rope_ref", wrong_rope)
    with pytest.raises(AssertionError):
        test_qk_norm_rope_matches_hf_layers()


def test_product_flop_count_matches_oracle_and_brute_force():
    """The benchmark's FLOP formula (package) equals the oracle's and a brute-force pair count."""
    from nano_vllm_ascend_amd.workloads import causal_attention_flops
    from oracle.attention_ref import prefill_flops

    q_lens, kv_lens = [5, 1, 7, 3], [5, 9, 7, 11]
    pairs = sum(1 for ql, kl in zip(q_lens, kv_lens) for r in range(ql) for j in range(kl) if j <= kl - ql + r)
    assert causal_attention_flops(q_lens, kv_lens, 16) == prefill_flops(q_lens, kv_lens, 16) == 4 * 128 * 16 * pairs
