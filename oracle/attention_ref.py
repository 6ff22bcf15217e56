"""fp32 CPU restatement of the reference attention path (test infrastructure only).

Citations are relative to the nano_vllm_ascend tree ("nv/" = src/nanovllm_ascend/).

Pins (tests/test_oracle.py):
  paged_decode_ref      torch SDPA on the gathered K/V; brute-force loops on a
                        tiny case; equals the last row of causal prefill.
  varlen_prefill_ref    torch SDPA(is_causal, enable_gqa) per sequence; HF
                        transformers eager_attention_forward with repeat_kv.
  paged_prefill_ref     equals the matching rows of dense prefill over the
                        full prompt (the reference's cache-hit == no-cache
                        invariant); reduces to varlen_prefill_ref at q == kv.
  kv_write_ref          closed form; untouched slots keep their bytes.
  rope_cos_sin_table    same torch formula as the reference; RoPE at position
                        0 is the identity; (d, d+64) pairs keep their norm.
  qk_norm_rope_ref      HF Qwen3RMSNorm + apply_rotary_pos_emb within one bf16
                        ulp; RMS of the normed row equals 1 for unit weights.
"""
from __future__ import annotations

import torch


def _gather_paged(cache: torch.Tensor, block_row: torch.Tensor, length: int) -> torch.Tensor:
    """Rows [0, length) of one sequence, gathered through its block-table row: [length, Hkv, D]."""
    nb, bs, hkv, d = cache.shape
    nblk = (length + bs - 1) // bs
    blocks = block_row[:nblk].long()
    return cache[blocks].reshape(nblk * bs, hkv, d)[:length]


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, allowed: torch.Tensor | None):
    """q [Tq, Hq, D], k/v [Tk, Hkv, D] -> [Tq, Hq, D] fp32; GQA maps query head h to kv head h // (Hq/Hkv)."""
    hq, hkv = q.shape[1], k.shape[1]
    group = hq // hkv
    k = k.float().repeat_interleave(group, dim=1)
    v = v.float().repeat_interleave(group, dim=1)
    s = torch.einsum("qhd,khd->hqk", q.float(), k) * scale
    if allowed is not None:
        s = s.masked_fill(~allowed.unsqueeze(0), float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("hqk,khd->qhd", p, v)


def paged_decode_ref(q, key_cache, value_cache, block_tables, context_lens, scale):
    """GQA paged decode (nv/layers/npu_paged_attention.py:27-100 semantics).

    For decode token i and query head h: softmax(q[i,h] . K^T * scale) V over the
    first context_lens[i] positions of sequence i, K/V gathered through
    block_tables[i] (context_lens includes the current token).
    """
    q = q.cpu()
    key_cache, value_cache = key_cache.cpu(), value_cache.cpu()
    block_tables, context_lens = block_tables.cpu(), context_lens.cpu()
    out = torch.zeros(q.shape, dtype=torch.float32)
    for i in range(q.shape[0]):
        ctx = int(context_lens[i])
        if ctx <= 0:
            continue
        k = _gather_paged(key_cache, block_tables[i], ctx)
        v = _gather_paged(value_cache, block_tables[i], ctx)
        out[i] = _attend(q[i : i + 1], k, v, scale, None)[0]
    return out


def varlen_prefill_ref(q, k, v, cu_seqlens, scale):
    """Dense causal varlen prefill (nv/layers/npu_prefill_attention.py:98-112, sparse_mode=3).

    Packed TND layout; sequence s owns rows cu_seqlens[s]:cu_seqlens[s+1]; row i
    of a sequence sees rows 0..i of the same sequence.
    """
    q, k, v = q.cpu(), k.cpu(), v.cpu()
    out = torch.zeros(q.shape, dtype=torch.float32)
    cu = [int(x) for x in cu_seqlens]
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        n = b - a
        if n <= 0:
            continue
        allowed = torch.ones(n, n, dtype=torch.bool).tril()
        out[a:b] = _attend(q[a:b], k[a:b], v[a:b], scale, allowed)
    return out


def paged_prefill_ref(q, key_cache, value_cache, block_tables, cu_seqlens_q, kv_lens, scale):
    """Prefix-hit prefill through the cache (nv/layers/npu_prefill_attention.py:66-96).

    Sequence s has q_len = cu[s+1]-cu[s] query rows and kv_len = kv_lens[s] keys
    read through block_tables[s]; causality is bottom-right aligned: query row r
    sees keys j <= kv_len - q_len + r.
    """
    q = q.cpu()
    key_cache, value_cache = key_cache.cpu(), value_cache.cpu()
    block_tables = block_tables.cpu()
    out = torch.zeros(q.shape, dtype=torch.float32)
    cu = [int(x) for x in cu_seqlens_q]
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        ql, kl = b - a, int(kv_lens[s])
        if ql <= 0:
            continue
        k = _gather_paged(key_cache, block_tables[s], kl)
        v = _gather_paged(value_cache, block_tables[s], kl)
        rows = torch.arange(ql).unsqueeze(1)
        cols = torch.arange(kl).unsqueeze(0)
        allowed = cols <= (kl - ql + rows)
        out[a:b] = _attend(q[a:b], k, v, scale, allowed)
    return out


def kv_write_ref(key_states, value_states, key_cache, value_cache, slot_mapping):
    """PagedKVCache.write (nv/npu/paged_kv_cache.py:44-69): index_copy_ into the flattened cache.

    Returns new (key_cache, value_cache) CPU tensors; negative slots are skipped
    (padding rows, an extension the reference never emits).
    """
    kc, vc = key_cache.cpu().clone(), value_cache.cpu().clone()
    nb, bs, hkv, d = kc.shape
    slots = slot_mapping.cpu().long()
    keep = slots >= 0
    kc.view(nb * bs, hkv, d).index_copy_(0, slots[keep], key_states.cpu()[keep].to(kc.dtype))
    vc.view(nb * bs, hkv, d).index_copy_(0, slots[keep], value_states.cpu()[keep].to(vc.dtype))
    return kc, vc


def rope_cos_sin_table(head_dim: int, max_positions: int, theta: float):
    """The reference's fp32 cos/sin cache (nv/layers/rotary_embedding.py:20-42).

    inv_freq = 1 / theta^(arange(0, D, 2)/D); freqs = outer(pos, inv_freq);
    emb = cat(freqs, freqs); returns (cos(emb), sin(emb)) as [max_positions, D].
    """
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    pos = torch.arange(max_positions, dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def rms_norm_head_ref(x, weight, eps):
    """npu_rms_norm per head (nv/layers/layernorm.py:12-17): fp32 x*rsqrt(mean(x^2)+eps)*w, one bf16 rounding."""
    xf = x.cpu().float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    return (xf * torch.rsqrt(var + eps) * weight.cpu().float()).to(torch.bfloat16)


def rope_ref(x, cos, sin):
    """npu_rotary_mul(rotary_mode="half") on bf16 x with bf16 cos/sin (nv/layers/rotary_embedding.py:78-97).

    x [T, H, D]; cos/sin [T, D] fp32, rounded to bf16 as the reference does
    (cos.to(q.dtype)); rotation in fp32, one bf16 rounding.
    """
    half = x.shape[-1] // 2
    xf = x.cpu().float()
    c = cos.cpu().to(torch.bfloat16).float().unsqueeze(1)
    s = sin.cpu().to(torch.bfloat16).float().unsqueeze(1)
    rot = torch.cat((-xf[..., half:], xf[..., :half]), dim=-1)
    return (xf * c + rot * s).to(torch.bfloat16)


def qk_norm_rope_ref(q, k, q_weight, k_weight, positions, theta, eps, max_positions=None):
    """Qwen3Attention.forward steps 2-3 (nv/models/qwen3.py:83-89): per-head norms, then RoPE."""
    pos = positions.cpu().long()
    mp = max_positions or int(pos.max()) + 1
    cos_t, sin_t = rope_cos_sin_table(q.shape[-1], mp, theta)
    cos, sin = cos_t.index_select(0, pos), sin_t.index_select(0, pos)
    qn = rms_norm_head_ref(q, q_weight, eps)
    kn = rms_norm_head_ref(k, k_weight, eps)
    return rope_ref(qn, cos, sin), rope_ref(kn, cos, sin)


def decode_bytes(context_lens, num_heads, num_kv_heads, head_dim=128, bt_width=0, elem=2) -> int:
    """Algorithmic HBM bytes of one paged decode launch.

    K and V read once per kv head and context token, q read and out written
    once, plus the block-table rows and context_lens.
    """
    ctx = int(sum(int(c) for c in context_lens))
    b = len(context_lens)
    return ctx * num_kv_heads * head_dim * elem * 2 + 2 * b * num_heads * head_dim * elem + b * bt_width * 4 + b * 4


def prefill_flops(q_lens, kv_lens, num_heads, head_dim=128) -> float:
    """Causal attention FLOPs: 4*D*Hq per visible (query, key) pair (QK^T and PV)."""
    pairs = 0
    for ql, kl in zip(q_lens, kv_lens):
        # query row r sees kl - ql + r + 1 keys
        pairs += ql * (kl - ql) + ql * (ql + 1) // 2
    return 4.0 * head_dim * num_heads * pairs


def scale_for(head_dim: int) -> float:
    return head_dim ** -0.5


__all__ = [
    "paged_decode_ref",
    "varlen_prefill_ref",
    "paged_prefill_ref",
    "kv_write_ref",
    "rope_cos_sin_table",
    "rms_norm_head_ref",
    "rope_ref",
    "qk_norm_rope_ref",
    "decode_bytes",
    "prefill_flops",
    "scale_for",
]
