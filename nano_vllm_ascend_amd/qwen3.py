"""Qwen3 decoder with the HIP attention path (nv/models/qwen3.py:1-221).

Per layer: RMSNorm -> fused qkv projection -> per-head RMSNorm of q and k, rotate-half
RoPE and the KV store of post-RoPE k and raw v -> prefill or paged-decode attention ->
o_proj -> residual -> RMSNorm -> SwiGLU MLP (fused gate/up projection) -> residual.
Prefill runs the norm/RoPE/store as one kernel (qk_norm_rope) before attention; a decode
batch runs all of it inside the paged-decode launch (one kernel, identical bits).  q/k/v
are views into the fused projection output, which the kernels accept through their row
strides.

Decode batches of <= 128 rows take a fused path (``forward_decode_fused``): the
skinny-M HIP GEMM runs every projection, each RMSNorm in the prologue of the GEMM
that consumes it, and each residual add in the epilogue of the GEMM that produces
it (with the per-32-column sums of squares the next norm needs), and SiLU*mul in
the gate/up epilogue -- 5 launches per layer instead of 9, same rounding points.
That path reads tiled copies of the projection weights (the GEMM's operand order,
built once by ``build_decode_weights``) and keeps the residual stream and the SiLU
output tiled as well; the qkv output, the attention output and the logits stay
row-major.  Prefill and larger batches run the unfused chain on hipBLASLt +
add_rms_norm over the row-major weights.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import nn

from . import _C
from .config import Qwen3Config
from .layers import (HipBatchPrefillAttention, HipPagedAttention, RMSNorm, RotaryEmbedding, gate_up_silu, linear,
                     qk_norm_rope)


@dataclass
class CausalLMOutput:
    logits: torch.Tensor


class Qwen3Attention(nn.Module):
    def __init__(self, config: Qwen3Config, layer_idx: int, block_size: int, max_model_len: int):
        super().__init__()
        self.layer_idx = layer_idx
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_weight = nn.Parameter(torch.empty(self.q_size + 2 * self.kv_size, config.hidden_size))
        self.o_weight = nn.Parameter(torch.empty(config.hidden_size, self.q_size))
        self.q_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.k_norm = RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.prefill_attn = HipBatchPrefillAttention(self.num_heads, self.num_kv_heads, self.head_dim, block_size,
                                                     max_model_len)
        self.paged_attn = HipPagedAttention(self.num_heads, self.num_kv_heads, self.head_dim)
        self.qkv_tiled = None  # tiled copies for the fused decode path (build_tiled)
        self.o_tiled = None

    def build_tiled(self) -> None:
        self.qkv_tiled = _C.tile(self.qkv_weight.detach())
        self.o_tiled = _C.tile(self.o_weight.detach())

    def forward(self, hidden_states, rotary: RotaryEmbedding, positions, kv_cache, attn_metadata, is_prefill: bool):
        t = hidden_states.shape[0]
        qkv = linear(hidden_states, self.qkv_weight, tiled=self.qkv_tiled)
        q = qkv[:, : self.q_size].view(t, self.num_heads, self.head_dim)
        k = qkv[:, self.q_size : self.q_size + self.kv_size].view(t, self.num_kv_heads, self.head_dim)
        v = qkv[:, self.q_size + self.kv_size :].view(t, self.num_kv_heads, self.head_dim)
        if is_prefill:
            qk_norm_rope(q, k, v, self.q_norm, self.k_norm, rotary, positions, kv_cache, self.layer_idx,
                         attn_metadata.slot_mapping)
            key_cache, value_cache = kv_cache.get_physical_cache(self.layer_idx)
            attn = self.prefill_attn(q, k, v, attn_metadata, key_cache, value_cache)
        else:
            attn = self.decode_attention(q, k, v, rotary, positions, kv_cache, attn_metadata)
        return linear(attn.reshape(t, self.q_size), self.o_weight, skinny=False)

    def decode_attention(self, q, k, v, rotary, positions, kv_cache, attn_metadata):
        """q/k norms, RoPE, the KV store and paged attention of a decode batch in one launch."""
        key_cache, value_cache = kv_cache.get_physical_cache(self.layer_idx)
        return self.paged_attn.decode_step(q, k, v, self.q_norm, self.k_norm, rotary, positions, key_cache,
                                           value_cache, attn_metadata.slot_mapping, attn_metadata.block_tables,
                                           attn_metadata.context_lens,
                                           max_context_len=getattr(attn_metadata, "max_context_bound", None),
                                           workspace=getattr(attn_metadata, "decode_workspace", None))

    def decode_fused(self, residual, ssq, t: int, norm: RMSNorm, rotary, positions, kv_cache, attn_metadata,
                     workspace):
        """residual += o_proj(attention(qkv_proj(norm(residual)))) in place, for a decode batch of
        t <= 128 rows held tiled in `residual`: the input RMSNorm runs in the qkv GEMM's prologue and
        the residual add (with the sums of squares the next norm needs) in the o_proj GEMM's epilogue."""
        qkv = _C.skinny_linear(residual, self.qkv_tiled, x_ssq=ssq, norm_weight=norm.weight,
                               eps=norm.variance_epsilon, workspace=workspace, m=t)
        q = qkv[:, : self.q_size].view(t, self.num_heads, self.head_dim)
        k = qkv[:, self.q_size : self.q_size + self.kv_size].view(t, self.num_kv_heads, self.head_dim)
        v = qkv[:, self.q_size + self.kv_size :].view(t, self.num_kv_heads, self.head_dim)
        attn = self.decode_attention(q, k, v, rotary, positions, kv_cache, attn_metadata)
        _C.skinny_linear(attn.reshape(t, self.q_size), self.o_tiled, residual, epilogue=_C.EPI_RESID, y_ssq=ssq,
                         workspace=workspace, y_tiled=True)


class Qwen3MLP(nn.Module):
    def __init__(self, config: Qwen3Config):
        super().__init__()
        self.intermediate = config.intermediate_size
        self.gate_up_weight = nn.Parameter(torch.empty(2 * config.intermediate_size, config.hidden_size))
        self.down_weight = nn.Parameter(torch.empty(config.hidden_size, config.intermediate_size))
        self.gate_up_tiled = None  # tiled copies for the fused decode path (build_tiled)
        self.down_tiled = None

    def build_tiled(self) -> None:
        self.gate_up_tiled = _C.tile(self.gate_up_weight.detach())
        self.down_tiled = _C.tile(self.down_weight.detach())

    def forward(self, x):
        return linear(gate_up_silu(x, self.gate_up_weight, self.gate_up_tiled), self.down_weight, skinny=False)

    def decode_fused(self, residual, ssq, t: int, norm: RMSNorm, workspace):
        """residual += down(silu(gate(norm(residual))) * up(norm(residual))) in place (t <= 128 rows,
        tiled): norm in the gate/up GEMM's prologue, SiLU*mul in its epilogue (written tiled), the
        residual add in the down GEMM's epilogue."""
        act = _C.skinny_linear(residual, self.gate_up_tiled, epilogue=_C.EPI_SILU, x_ssq=ssq,
                               norm_weight=norm.weight, eps=norm.variance_epsilon, workspace=workspace, m=t,
                               y_tiled=True)
        _C.skinny_linear(act, self.down_tiled, residual, epilogue=_C.EPI_RESID, y_ssq=ssq, workspace=workspace, m=t,
                         y_tiled=True)


class Qwen3DecoderLayer(nn.Module):
    def __init__(self, config: Qwen3Config, layer_idx: int, block_size: int, max_model_len: int):
        super().__init__()
        self.self_attn = Qwen3Attention(config, layer_idx, block_size, max_model_len)
        self.mlp = Qwen3MLP(config)
        self.input_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, h, rotary, positions, kv_cache, attn_metadata, is_prefill):
        h = h + self.self_attn(self.input_layernorm(h), rotary, positions, kv_cache, attn_metadata, is_prefill)
        return h + self.mlp(self.post_attention_layernorm(h))


class Qwen3Model(nn.Module):
    def __init__(self, config: Qwen3Config, block_size: int, max_model_len: int):
        super().__init__()
        self.embed_tokens = nn.Parameter(torch.empty(config.vocab_size, config.hidden_size))
        self.layers = nn.ModuleList(
            [Qwen3DecoderLayer(config, i, block_size, max_model_len) for i in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(config.head_dim, config.max_position_embeddings, config.rope_theta)

    def forward(self, input_ids_flat, position_ids_flat, kv_cache, attn_metadata, is_prefill):
        # The residual stream lives in one buffer updated in place; every "residual + h" and the
        # RMSNorm that follows it is one add_rms_norm launch (same bf16 rounding as the reference).
        residual = F.embedding(input_ids_flat, self.embed_tokens)
        x = self.layers[0].input_layernorm(residual)
        n = len(self.layers)
        for i, layer in enumerate(self.layers):
            a = layer.self_attn(x, self.rotary_emb, position_ids_flat, kv_cache, attn_metadata, is_prefill)
            layer.post_attention_layernorm.add_forward(a, residual, x)
            m = layer.mlp(x)
            nxt = self.layers[i + 1].input_layernorm if i + 1 < n else self.norm
            nxt.add_forward(m, residual, x)
        return x

    def forward_decode_fused(self, input_ids_flat, position_ids_flat, kv_cache, attn_metadata, workspace):
        """Decode forward for <= 128 rows with every RMSNorm and residual add folded into the
        projections: 5 launches per layer (qkv, norm/RoPE/store + attention, o, gate_up, down).
        Returns the final residual stream (tiled, 16 * ceil(t/16) rows) and its per-32-column sums
        of squares; the final norm runs in the LM head's prologue."""
        t = input_ids_flat.shape[0]
        hidden = self.embed_tokens.shape[1]
        ssq = torch.empty((t, hidden // 32), dtype=torch.float32, device=self.embed_tokens.device)
        residual = _C.embed_rows(input_ids_flat, self.embed_tokens, ssq=ssq, out_tiled=True)
        for layer in self.layers:
            layer.self_attn.decode_fused(residual, ssq, t, layer.input_layernorm, self.rotary_emb, position_ids_flat,
                                         kv_cache, attn_metadata, workspace)
            layer.mlp.decode_fused(residual, ssq, t, layer.post_attention_layernorm, workspace)
        return residual, ssq


class Qwen3ForCausalLM(nn.Module):
    def __init__(self, config: Qwen3Config, block_size: int = 128, max_model_len: int = 2048):
        super().__init__()
        self.config = config
        self.model = Qwen3Model(config, block_size, max_model_len)
        self.lm_head = self.model.embed_tokens if config.tie_word_embeddings else nn.Parameter(
            torch.empty(config.vocab_size, config.hidden_size))

        self._gemm_workspace = None
        self.lm_head_tiled = None
        self._tiled_ready = False

    def build_decode_weights(self) -> None:
        """Tiled copies of the projection and LM head weights for the fused decode path (about the
        size of the weights again).  Built on the first fused decode; call it again after changing
        weights in place."""
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the tiled decode weights must be built before graph capture")
        for layer in self.model.layers:
            layer.self_attn.build_tiled()
            layer.mlp.build_tiled()
        self.lm_head_tiled = _C.tile(self.lm_head.detach())
        self._tiled_ready = True

    def _drop_decode_weights(self) -> None:
        """Forget the tiled copies (the weights are about to change)."""
        for layer in self.model.layers:
            layer.self_attn.qkv_tiled = layer.self_attn.o_tiled = None
            layer.mlp.gate_up_tiled = layer.mlp.down_tiled = None
        self.lm_head_tiled = None
        self._tiled_ready = False

    def decode_fusable(self, rows: int) -> bool:
        """Whether a decode batch of `rows` runs on the fused skinny-GEMM path."""
        c = self.config
        dev = self.model.embed_tokens.device
        return (dev.type == "cuda" and 0 < rows <= _C.SKINNY_MAX_ROWS and c.hidden_size % 1024 == 0
                and c.hidden_size <= 2048 and c.intermediate_size % 256 == 0
                and (c.num_attention_heads * c.head_dim) % 256 == 0 and c.vocab_size % 32 == 0)

    def gemm_workspace(self) -> torch.Tensor:
        """Zero-filled workspace shared by the decode projections (calls run in stream order)."""
        if self._gemm_workspace is None:
            c = self.config
            h, i, q = c.hidden_size, c.intermediate_size, c.num_attention_heads * c.head_dim
            shapes = [(h, q, _C.EPI_RESID), (h, i, _C.EPI_RESID), (i, h, _C.EPI_SILU),
                      (q + 2 * c.num_key_value_heads * c.head_dim, h, _C.EPI_STORE), (c.vocab_size, h, _C.EPI_STORE)]
            need = max([_C.skinny_linear_workspace_size(n, k, e) for n, k, e in shapes] + [16])
            self._gemm_workspace = torch.zeros(need, dtype=torch.uint8, device=self.model.embed_tokens.device)
        return self._gemm_workspace

    def forward(self, input_ids_flat, position_ids_flat, kv_cache, attn_metadata, is_prefill: bool,
                logits_indices=None) -> CausalLMOutput:
        if not is_prefill and logits_indices is None and self.decode_fusable(input_ids_flat.shape[0]):
            if not self._tiled_ready or self.lm_head_tiled.device != self.lm_head.device:
                self.build_decode_weights()
            ws = self.gemm_workspace()
            residual, ssq = self.model.forward_decode_fused(input_ids_flat, position_ids_flat, kv_cache,
                                                            attn_metadata, ws)
            norm = self.model.norm
            return CausalLMOutput(logits=_C.skinny_linear(residual, self.lm_head_tiled, x_ssq=ssq,
                                                          norm_weight=norm.weight, eps=norm.variance_epsilon,
                                                          workspace=ws, m=input_ids_flat.shape[0]))
        h = self.model(input_ids_flat, position_ids_flat, kv_cache, attn_metadata, is_prefill)
        if logits_indices is not None:
            h = h.index_select(0, logits_indices)
        return CausalLMOutput(logits=linear(h, self.lm_head, tiled=self.lm_head_tiled))

    # ---------------------------------------------------------------- weights
    @torch.no_grad()
    def init_random(self, seed: int = 0, std: float | None = None) -> None:
        """Seeded N(0, std) for every projection and the embedding, ones for every norm weight."""
        std = self.config.initializer_range if std is None else std
        self._drop_decode_weights()
        dev = self.model.embed_tokens.device
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.fill_(1.0)
            else:
                tmp = torch.empty(p.shape, dtype=torch.float32, device=dev)
                tmp.normal_(0.0, std, generator=gen)
                p.copy_(tmp)

    @torch.no_grad()
    def load_hf_state_dict(self, sd: dict) -> list[str]:
        """Copy HF Qwen3ForCausalLM weights (q/k/v and gate/up are concatenated); returns missing names."""
        missing = []
        self._drop_decode_weights()
        m = self.model

        def put(dst, name):
            if name in sd:
                dst.copy_(sd[name])
            else:
                missing.append(name)

        put(m.embed_tokens, "model.embed_tokens.weight")
        put(m.norm.weight, "model.norm.weight")
        for i, layer in enumerate(m.layers):
            p = f"model.layers.{i}."
            a = layer.self_attn
            names = [p + "self_attn.q_proj.weight", p + "self_attn.k_proj.weight", p + "self_attn.v_proj.weight"]
            if all(n in sd for n in names):
                a.qkv_weight.copy_(torch.cat([sd[n] for n in names], 0))
            else:
                missing += [n for n in names if n not in sd]
            put(a.o_weight, p + "self_attn.o_proj.weight")
            put(a.q_norm.weight, p + "self_attn.q_norm.weight")
            put(a.k_norm.weight, p + "self_attn.k_norm.weight")
            names = [p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"]
            if all(n in sd for n in names):
                layer.mlp.gate_up_weight.copy_(torch.cat([sd[n] for n in names], 0))
            else:
                missing += [n for n in names if n not in sd]
            put(layer.mlp.down_weight, p + "mlp.down_proj.weight")
            put(layer.input_layernorm.weight, p + "input_layernorm.weight")
            put(layer.post_attention_layernorm.weight, p + "post_attention_layernorm.weight")
        if not self.config.tie_word_embeddings:
            put(self.lm_head, "lm_head.weight")
        return missing


def load_safetensors_dir(path) -> dict | None:
    """All tensors of the *.safetensors files in a local directory (safe loader; no pickle), or None."""
    files = sorted(Path(path).glob("*.safetensors")) if Path(path).is_dir() else []
    if not files:
        return None
    from safetensors.torch import load_file

    sd = {}
    for f in files:
        sd.update(load_file(str(f)))
    return sd
