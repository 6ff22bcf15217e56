"""CPU restatement of the reference Qwen3 forward (test infrastructure only).

Follows nv/models/qwen3.py:26-221 for one sequence at a time with a dense
per-layer KV cache: embedding -> per layer [RMSNorm -> q/k/v projections ->
per-head q/k RMSNorm -> rotate-half RoPE -> causal GQA attention -> o_proj ->
residual -> RMSNorm -> SwiGLU MLP -> residual] -> RMSNorm -> tied LM head.

round_bf16=True rounds every activation to bf16 where the reference's bf16
model produces a tensor (projection outputs, norm outputs, RoPE output,
attention output, residual sums, MLP intermediates); False keeps fp32
throughout.  Weights are given as a state dict of this repository's
Qwen3ForCausalLM (fused qkv / gate_up layout).

Pins (tests/test_oracle.py): in fp32 mode the logits equal HF transformers'
Qwen3ForCausalLM (eager attention) built from the same weights.
"""
from __future__ import annotations

import torch

from .attention_ref import rope_cos_sin_table


class Qwen3Ref:
    def __init__(self, state: dict, config, round_bf16: bool = True, max_positions: int = 4096, device="cpu"):
        """``device``: where the fp32 arithmetic runs (the CPU, or a GPU for the full-depth model)."""
        self.cfg = config
        self.rb = round_bf16
        self.device = torch.device(device)
        self.w = {k: v.detach().to(self.device, torch.float32) for k, v in state.items()}
        cos, sin = rope_cos_sin_table(config.head_dim, max_positions, config.rope_theta)
        if round_bf16:  # the reference casts the fp32 table to the activation dtype
            cos, sin = cos.to(torch.bfloat16).float(), sin.to(torch.bfloat16).float()
        self.cos, self.sin = cos.to(self.device), sin.to(self.device)
        self.reset()

    def reset(self):
        n = self.cfg.num_hidden_layers
        shape = (0, self.cfg.num_key_value_heads, self.cfg.head_dim)
        self.k_cache = [torch.zeros(shape, device=self.device) for _ in range(n)]
        self.v_cache = [torch.zeros(shape, device=self.device) for _ in range(n)]
        self.pos = 0

    def _r(self, x):
        return x.to(torch.bfloat16).float() if self.rb else x

    def _norm(self, x, w):
        var = x.pow(2).mean(-1, keepdim=True)
        return self._r(x * torch.rsqrt(var + self.cfg.rms_norm_eps) * w)

    def _rope(self, x, pos):
        half = x.shape[-1] // 2
        c = self.cos[pos].unsqueeze(1)
        s = self.sin[pos].unsqueeze(1)
        rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
        return self._r(x * c + rot * s)

    @torch.no_grad()
    def forward(self, token_ids: list[int]) -> torch.Tensor:
        """Append tokens to the cache; return fp32 logits of the last one."""
        cfg, w = self.cfg, self.w
        t = len(token_ids)
        pos = torch.arange(self.pos, self.pos + t, device=self.device)
        h = w["model.embed_tokens"][torch.tensor(token_ids, device=self.device)]
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        qs, kvs = hq * d, hkv * d
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            x = self._norm(h, w[p + "input_layernorm.weight"])
            qkv = self._r(x @ w[p + "self_attn.qkv_weight"].T)
            q = qkv[:, :qs].view(t, hq, d)
            k = qkv[:, qs : qs + kvs].view(t, hkv, d)
            v = qkv[:, qs + kvs :].view(t, hkv, d)
            q = self._rope(self._norm(q, w[p + "self_attn.q_norm.weight"]), pos)
            k = self._rope(self._norm(k, w[p + "self_attn.k_norm.weight"]), pos)
            self.k_cache[i] = torch.cat([self.k_cache[i], k])
            self.v_cache[i] = torch.cat([self.v_cache[i], v])
            kk = self.k_cache[i].repeat_interleave(hq // hkv, dim=1)
            vv = self.v_cache[i].repeat_interleave(hq // hkv, dim=1)
            # [h, q, d] @ [h, d, k] and [h, q, k] @ [h, k, d], contiguous fp32 operands
            s = torch.matmul(q.transpose(0, 1).contiguous(), kk.permute(1, 2, 0).contiguous()) * d ** -0.5
            keys = torch.arange(kk.shape[0], device=self.device)
            s = s.masked_fill(keys[None, None, :] > pos[None, :, None], float("-inf"))
            pv = torch.matmul(torch.softmax(s, -1), vv.transpose(0, 1).contiguous())
            a = self._r(pv.transpose(0, 1)).reshape(t, qs)
            h = self._r(h + self._r(a @ w[p + "self_attn.o_weight"].T))
            x = self._norm(h, w[p + "post_attention_layernorm.weight"])
            gu = self._r(x @ w[p + "mlp.gate_up_weight"].T)
            inter = cfg.intermediate_size
            act = self._r(self._r(torch.nn.functional.silu(gu[:, :inter])) * gu[:, inter:])
            h = self._r(h + self._r(act @ w[p + "mlp.down_weight"].T))
        h = self._norm(h, w["model.norm.weight"])
        self.pos += t
        head = w["model.embed_tokens"] if cfg.tie_word_embeddings else w["lm_head"]
        return h[-1] @ head.T


def load_into_hf(state: dict, hf_model, config) -> None:
    """Copy a fused-layout state dict into an HF Qwen3ForCausalLM (for the oracle's library cross-check)."""
    sd = {}
    qs = config.num_attention_heads * config.head_dim
    kvs = config.num_key_value_heads * config.head_dim
    inter = config.intermediate_size
    sd["model.embed_tokens.weight"] = state["model.embed_tokens"]
    sd["model.norm.weight"] = state["model.norm.weight"]
    for i in range(config.num_hidden_layers):
        p = f"model.layers.{i}."
        qkv = state[p + "self_attn.qkv_weight"]
        sd[p + "self_attn.q_proj.weight"] = qkv[:qs]
        sd[p + "self_attn.k_proj.weight"] = qkv[qs : qs + kvs]
        sd[p + "self_attn.v_proj.weight"] = qkv[qs + kvs :]
        sd[p + "self_attn.o_proj.weight"] = state[p + "self_attn.o_weight"]
        sd[p + "self_attn.q_norm.weight"] = state[p + "self_attn.q_norm.weight"]
        sd[p + "self_attn.k_norm.weight"] = state[p + "self_attn.k_norm.weight"]
        gu = state[p + "mlp.gate_up_weight"]
        sd[p + "mlp.gate_proj.weight"] = gu[:inter]
        sd[p + "mlp.up_proj.weight"] = gu[inter:]
        sd[p + "mlp.down_proj.weight"] = state[p + "mlp.down_weight"]
        sd[p + "input_layernorm.weight"] = state[p + "input_layernorm.weight"]
        sd[p + "post_attention_layernorm.weight"] = state[p + "post_attention_layernorm.weight"]
    sd["lm_head.weight"] = state["model.embed_tokens"]
    hf_model.load_state_dict({k: v.float() for k, v in sd.items()}, strict=False)
