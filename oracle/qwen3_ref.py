"""CPU restatement of the reference Qwen3 forward (test infrastructure only).

Follows nv/models/qwen3.py:26-221 for one sequence at a time with a dense
per-layer KV cache: embedding -> per layer [RMSNorm -> q/k/v projections ->
per-head q/k RMSNorm -> rotate-half RoPE -> causal GQA attention -> o_proj ->
residual -> RMSNorm -> SwiGLU MLP -> residual] -> RMSNorm -> tied LM head.

round_bf16=True rounds every activation to bf16 where the reference's bf16
model produces a tensor (projection outputs, norm outputs, RoPE output,
attention output, residual sums, MLP intermediates, and the logits: the
reference's LMHead is a bf16 linear, nv/layers/embed_head.py:34-39, and its
greedy sampler takes torch.argmax of that bf16 tensor, nv/layers/sampler.py:13-14,
so the first of equal bf16 logits wins); False keeps fp32 throughout.  Weights
are given as a state dict of this repository's Qwen3ForCausalLM (fused qkv /
gate_up layout).

Two further legal ways to evaluate the same bf16 model, used to measure how far
two correct implementations' greedy tokens drift apart:
  dtype=torch.float64   every product and sum in fp64 (same rounding points);
  round_probs=True      softmax probabilities rounded to bf16 before the PV
                        product, as a kernel that runs PV on a bf16 matrix unit does.

Pins (tests/test_oracle.py): in fp32 mode the logits equal HF transformers'
Qwen3ForCausalLM (eager attention) built from the same weights; fp64 mode agrees
with fp32 mode to fp32 rounding before any bf16 rounding point is crossed.
"""
from __future__ import annotations

import torch

from .attention_ref import rope_cos_sin_table


class Qwen3Ref:
    def __init__(self, state: dict, config, round_bf16: bool = True, max_positions: int = 4096, device="cpu",
                 dtype=torch.float32, round_probs: bool = False):
        """``device``: where the arithmetic runs (the CPU, or a GPU for the full-depth model);
        ``dtype``: its precision (float32, or float64 for a second evaluation order)."""
        self.cfg = config
        self.rb = round_bf16
        self.rp = round_probs
        self.dt = dtype
        self.device = torch.device(device)
        self.w = {k: v.detach().to(self.device, dtype) for k, v in state.items()}
        cos, sin = rope_cos_sin_table(config.head_dim, max_positions, config.rope_theta)
        if round_bf16:  # the reference casts the fp32 table to the activation dtype
            cos, sin = cos.to(torch.bfloat16).float(), sin.to(torch.bfloat16).float()
        self.cos, self.sin = cos.to(self.device, dtype), sin.to(self.device, dtype)
        self.reset()

    def reset(self, batch: int = 1):
        """Empty caches for `batch` sequences that advance together (``forward_batch``)."""
        n = self.cfg.num_hidden_layers
        shape = (batch, 0, self.cfg.num_key_value_heads, self.cfg.head_dim)
        self.k_cache = [torch.zeros(shape, device=self.device, dtype=self.dt) for _ in range(n)]
        self.v_cache = [torch.zeros(shape, device=self.device, dtype=self.dt) for _ in range(n)]
        self.batch = batch
        self.pos = 0

    def _r(self, x):
        return x.to(torch.bfloat16).to(self.dt) if self.rb else x

    def _norm(self, x, w):
        var = x.pow(2).mean(-1, keepdim=True)
        return self._r(x * torch.rsqrt(var + self.cfg.rms_norm_eps) * w)

    def _rope(self, x, pos):
        """x [B, t, heads, d], pos [t]."""
        half = x.shape[-1] // 2
        c = self.cos[pos][None, :, None, :]
        s = self.sin[pos][None, :, None, :]
        rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
        return self._r(x * c + rot * s)

    @torch.no_grad()
    def forward(self, token_ids: list[int]) -> torch.Tensor:
        """Append tokens to the cache of one sequence; return the logits of the last one."""
        if self.batch != 1:
            self.reset(1)
        return self._forward(torch.tensor([token_ids], device=self.device))[0]

    @torch.no_grad()
    def forward_batch(self, token_ids: list[list[int]]) -> torch.Tensor:
        """Append the same number of tokens to each of `batch` sequences that sit at the same
        position (equal-length prompts, then one token each); return [batch, vocab] logits of
        their last tokens.  Each sequence attends to its own cache only."""
        if len(token_ids) != self.batch or len({len(t) for t in token_ids}) != 1:
            raise ValueError("forward_batch takes one equal-length token list per sequence of reset(batch)")
        return self._forward(torch.tensor(token_ids, device=self.device))

    def _forward(self, ids: torch.Tensor) -> torch.Tensor:
        cfg, w = self.cfg, self.w
        bsz, t = ids.shape
        pos = torch.arange(self.pos, self.pos + t, device=self.device)
        h = w["model.embed_tokens"][ids]  # [B, t, hidden]
        hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        qs, kvs = hq * d, hkv * d
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."
            x = self._norm(h, w[p + "input_layernorm.weight"])
            qkv = self._r(x @ w[p + "self_attn.qkv_weight"].T)
            q = qkv[..., :qs].reshape(bsz, t, hq, d)
            k = qkv[..., qs : qs + kvs].reshape(bsz, t, hkv, d)
            v = qkv[..., qs + kvs :].reshape(bsz, t, hkv, d)
            q = self._rope(self._norm(q, w[p + "self_attn.q_norm.weight"]), pos)
            k = self._rope(self._norm(k, w[p + "self_attn.k_norm.weight"]), pos)
            self.k_cache[i] = torch.cat([self.k_cache[i], k], dim=1)
            self.v_cache[i] = torch.cat([self.v_cache[i], v], dim=1)
            kk = self.k_cache[i].repeat_interleave(hq // hkv, dim=2)  # [B, T, hq, d]
            vv = self.v_cache[i].repeat_interleave(hq // hkv, dim=2)
            # [B, h, q, d] @ [B, h, d, k] and [B, h, q, k] @ [B, h, k, d], contiguous operands
            s = torch.matmul(q.transpose(1, 2).contiguous(), kk.permute(0, 2, 3, 1).contiguous()) * d ** -0.5
            keys = torch.arange(kk.shape[1], device=self.device)
            s = s.masked_fill(keys[None, None, None, :] > pos[None, None, :, None], float("-inf"))
            probs = torch.softmax(s, -1)
            if self.rp:
                probs = probs.to(torch.bfloat16).to(self.dt)
            pv = torch.matmul(probs, vv.transpose(1, 2).contiguous())  # [B, h, t, d]
            a = self._r(pv.transpose(1, 2)).reshape(bsz, t, qs)
            h = self._r(h + self._r(a @ w[p + "self_attn.o_weight"].T))
            x = self._norm(h, w[p + "post_attention_layernorm.weight"])
            gu = self._r(x @ w[p + "mlp.gate_up_weight"].T)
            inter = cfg.intermediate_size
            act = self._r(self._r(torch.nn.functional.silu(gu[..., :inter])) * gu[..., inter:])
            h = self._r(h + self._r(act @ w[p + "mlp.down_weight"].T))
        h = self._norm(h, w["model.norm.weight"])
        self.pos += t
        head = w["model.embed_tokens"] if cfg.tie_word_embeddings else w["lm_head"]
        return self._r(h[:, -1] @ head.T).float()


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
