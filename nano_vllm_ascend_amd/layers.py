"""Model-runner-facing layers of the attention path (nv/layers/*).

Attention backends keep the reference's constructor and forward signatures
and raise ValueError on the same shape mismatches:
  HipPagedAttention        <- NpuPagedAttention        (nv/layers/npu_paged_attention.py:27-100)
  HipBatchPrefillAttention <- NpuBatchPrefillAttention (nv/layers/npu_prefill_attention.py:41-113)
The ``Npu*`` names are kept as aliases so code written against the reference
imports unchanged.  ``qk_norm_rope`` fuses q_norm, k_norm, RoPE and the KV
store (nv/models/qwen3.py:83-96) into one kernel.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from . import _C


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * w computed in fp32, one rounding to bf16 (nv/layers/layernorm.py).

    ``forward`` runs the HIP add_rms_norm kernel without the add; ``add_forward``
    fuses the decoder's residual add into the same launch.
    """

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x.contiguous()
        return _C.add_rms_norm(None, x, self.weight, torch.empty_like(x), self.variance_epsilon)

    def add_forward(self, delta: torch.Tensor, residual: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """residual += delta in place; out = norm(residual)."""
        return _C.add_rms_norm(delta, residual, self.weight, out, self.variance_epsilon)


class RotaryEmbedding(nn.Module):
    """The reference's fp32 cos/sin cache (nv/layers/rotary_embedding.py:8-62), stored for the fused kernel.

    The table is [max_position_embeddings, head_dim]: per position the 64 cos
    values then the 64 sin values of inv_freq = theta^(-2i/D) (the
    reference's emb = cat(freqs, freqs) repeats each half, so one half is kept).
    """

    def __init__(self, head_dim: int, max_position_embeddings: int = 40960, rope_theta: float = 1_000_000.0):
        super().__init__()
        self.head_dim = head_dim
        self.max_position_embeddings = max_position_embeddings
        self.rope_theta = rope_theta
        inv_freq = 1.0 / (rope_theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        freqs = torch.outer(torch.arange(max_position_embeddings, dtype=torch.float32), inv_freq)
        self.register_buffer("cos_sin", torch.cat((freqs.cos(), freqs.sin()), dim=1).contiguous(), persistent=False)


def qk_norm_rope(q, k, v, q_norm: RMSNorm, k_norm: RMSNorm, rotary: RotaryEmbedding, positions, kv_cache=None,
                 layer_idx: int = 0, slot_mapping=None) -> None:
    """In place: q, k <- RoPE(head RMSNorm); with a cache, also store post-RoPE k and raw v at slot_mapping."""
    kc = vc = None
    if kv_cache is not None:
        kc, vc = kv_cache.get_physical_cache(layer_idx)
    _C.qk_norm_rope(q, k, q_norm.weight, k_norm.weight, positions, rotary.cos_sin, q_norm.variance_epsilon,
                    v=v if kc is not None else None, key_cache=kc, value_cache=vc,
                    slot_mapping=slot_mapping if kc is not None else None)


class HipPagedAttention(nn.Module):
    """GQA paged decode attention over block_tables / context_lens (context_lens on the device)."""

    def __init__(self, num_heads: int, num_key_value_heads: int, head_dim: int):
        super().__init__()
        self.num_heads = num_heads
        self.num_key_value_heads = num_key_value_heads
        self.head_dim = head_dim
        self.scale = head_dim ** -0.5
        self._workspace: torch.Tensor | None = None
        self._ws_key = (0, 0)

    def workspace(self, batch: int, max_context_len: int, device) -> torch.Tensor:
        """A zero-filled split-KV workspace large enough for (batch, max_context_len); grows on demand."""
        b, c = self._ws_key
        if self._workspace is None or batch > b or max_context_len > c or self._workspace.device != device:
            b, c = max(batch, b), max(max_context_len, c)
            self._workspace = _C.alloc_paged_decode_workspace(b, self.num_heads, self.num_key_value_heads, c, device)
            self._ws_key = (b, c)
        return self._workspace

    def forward(self, q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                block_tables: torch.Tensor, context_lens: torch.Tensor, max_context_len: int | None = None,
                workspace: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        total_tokens, num_heads, head_dim = q.shape
        if num_heads != self.num_heads or head_dim != self.head_dim:
            raise ValueError(f"query shape mismatch: got {tuple(q.shape)}")
        if max_context_len is None:  # bound from the table width: no host sync needed
            max_context_len = block_tables.shape[1] * key_cache.shape[1]
        if context_lens.device != q.device:
            context_lens = context_lens.to(q.device, non_blocking=True)
        if workspace is None:
            workspace = self.workspace(total_tokens, max_context_len, q.device)
        out = torch.empty_like(q) if out is None else out
        return _C.paged_decode(out, q, key_cache, value_cache, block_tables, context_lens.to(torch.int32),
                               self.scale, max_context_len, workspace)


    def decode_step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm: RMSNorm, k_norm: RMSNorm,
                    rotary: RotaryEmbedding, positions: torch.Tensor, key_cache: torch.Tensor,
                    value_cache: torch.Tensor, slot_mapping: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor, max_context_len: int | None = None,
                    workspace: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """One launch for a decode batch: q/k RMSNorm + RoPE, the KV store of post-RoPE k and raw v at
        slot_mapping, then this attention -- bit-identical to qk_norm_rope followed by forward().
        q, k, v are the raw projection rows and are left unmodified."""
        total_tokens, num_heads, head_dim = q.shape
        if num_heads != self.num_heads or head_dim != self.head_dim:
            raise ValueError(f"query shape mismatch: got {tuple(q.shape)}")
        if max_context_len is None:
            max_context_len = block_tables.shape[1] * key_cache.shape[1]
        if context_lens.device != q.device:
            context_lens = context_lens.to(q.device, non_blocking=True)
        if workspace is None:
            workspace = self.workspace(total_tokens, max_context_len, q.device)
        out = torch.empty_like(q) if out is None else out
        return _C.paged_decode_fused(out, q, k, v, q_norm.weight, k_norm.weight, positions, rotary.cos_sin,
                                     q_norm.variance_epsilon, key_cache, value_cache, slot_mapping, block_tables,
                                     context_lens.to(torch.int32), self.scale, max_context_len, workspace)


class HipBatchPrefillAttention(nn.Module):
    """Causal varlen prefill; dense route on activations, paged route (any prefix hit) through the cache."""

    def __init__(self, num_heads: int, num_key_value_heads: int, head_dim: int, block_size: int, max_mask_len: int):
        super().__init__()
        self.num_heads = num_heads
        self.num_key_value_heads = num_key_value_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.max_mask_len = max_mask_len
        self.scale = head_dim ** -0.5

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_metadata,
                key_cache: torch.Tensor | None = None, value_cache: torch.Tensor | None = None) -> torch.Tensor:
        total_tokens, num_heads, head_dim = q.shape
        if num_heads != self.num_heads or head_dim != self.head_dim:
            raise ValueError(f"query shape mismatch: got {tuple(q.shape)}")
        if k.shape[0] != total_tokens or v.shape[0] != total_tokens:
            raise ValueError(f"k/v token mismatch: q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
        max_q = attn_metadata.max_query_len
        if not max_q and attn_metadata.actual_seq_lengths_q:
            ends = attn_metadata.actual_seq_lengths_q
            max_q = max(b - a for a, b in zip([0] + ends[:-1], ends))
        if max_q > self.max_mask_len:
            raise ValueError(f"prompt length {max_q} exceeds max_mask_len {self.max_mask_len}")
        out = torch.empty_like(q)
        if attn_metadata.use_paged_prefill:
            if key_cache is None or value_cache is None:
                raise ValueError("paged prefill requires physical key/value cache")
            return _C.paged_prefill(out, q, key_cache, value_cache, attn_metadata.block_tables,
                                    attn_metadata.cu_seqlens_q, attn_metadata.context_lens, max_q, self.scale)
        return _C.varlen_prefill(out, q, k, v, attn_metadata.cu_seqlens_q, max_q, self.scale)


NpuPagedAttention = HipPagedAttention
NpuBatchPrefillAttention = HipBatchPrefillAttention


class Sampler:
    """Greedy argmax, or temperature -> top-k -> top-p -> multinomial (nv/layers/sampler.py:8-48)."""

    def sample(self, logits: torch.Tensor, sampling_params) -> torch.Tensor:
        if logits.dim() != 2:
            raise ValueError(f"logits must have shape [batch, vocab], got {tuple(logits.shape)}")
        if sampling_params.is_greedy():
            return torch.argmax(logits, dim=-1)
        x = logits / sampling_params.temperature
        x = self._top_k(x, sampling_params.top_k)
        x = self._top_p(x, sampling_params.top_p)
        return torch.multinomial(torch.softmax(x, dim=-1), num_samples=1).squeeze(-1)

    @staticmethod
    def _top_k(x: torch.Tensor, k: int) -> torch.Tensor:
        if k <= 0 or k >= x.shape[-1]:
            return x
        kth = torch.topk(x, k=k, dim=-1).values[..., -1:]
        return x.masked_fill(x < kth, float("-inf"))

    @staticmethod
    def _top_p(x: torch.Tensor, p: float) -> torch.Tensor:
        if p >= 1.0:
            return x
        sorted_x, order = torch.sort(x, dim=-1, descending=True)
        cum = torch.softmax(sorted_x, dim=-1).cumsum(dim=-1)
        drop = cum > p
        drop[..., 1:] = drop[..., :-1].clone()  # keep the first token that crosses p
        drop[..., 0] = False
        out = x.clone()
        out.scatter_(-1, order, sorted_x.masked_fill(drop, float("-inf")))
        return out


def _skinny_ok(x: torch.Tensor, weight: torch.Tensor, tiled: torch.Tensor | None) -> bool:
    return (tiled is not None and x.is_cuda and x.dim() == 2 and 0 < x.shape[0] <= _C.SKINNY_MAX_ROWS
            and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and x.stride(1) == 1
            and weight.shape[0] % 32 == 0 and x.shape[1] % 256 == 0 and x.data_ptr() % 16 == 0
            and x.stride(0) % 8 == 0)


def linear(x: torch.Tensor, weight: torch.Tensor, skinny: bool = True,
           tiled: torch.Tensor | None = None) -> torch.Tensor:
    """x @ weight^T.  Batches of <= 128 rows use the skinny-M HIP kernel when the weight's tiled
    copy (``_C.tile(weight)``) is given -- it streams the weight once; otherwise, and for larger
    batches (prefill), the library GEMM.  ``skinny=False`` keeps a projection on the library GEMM."""
    if skinny and _skinny_ok(x, weight, tiled):
        return _C.linear(x, tiled)
    return F.linear(x, weight)


def gate_up_silu(x: torch.Tensor, w_gate_up: torch.Tensor, tiled: torch.Tensor | None = None) -> torch.Tensor:
    """silu(x @ W_gate^T) * (x @ W_up^T) for the fused [2I, H] weight (nv/models/qwen3.py:34-35):
    one HIP launch for batches of <= 128 rows when the weight's tiled copy is given, library GEMM +
    silu_mul kernel otherwise."""
    if _skinny_ok(x, w_gate_up, tiled) and (w_gate_up.shape[0] // 2) % 32 == 0:
        return _C.linear_silu_mul(x, tiled)
    return _C.silu_mul(F.linear(x, w_gate_up))
