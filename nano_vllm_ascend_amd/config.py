"""Qwen3 model configuration (the fields nv/models/qwen3.py reads from the HF config).

``load_config(model_path)`` accepts a directory holding an HF ``config.json``,
an existing ``Qwen3Config``, or a dict of overrides on the Qwen3-0.6B shape.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass, fields, replace
from pathlib import Path


@dataclass(frozen=True)
class Qwen3Config:
    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_position_embeddings: int = 40960
    tie_word_embeddings: bool = True
    attention_bias: bool = False
    eos_token_id: int = 151645
    initializer_range: float = 0.02

    def to_dict(self) -> dict:
        return asdict(self)


QWEN3_0_6B = Qwen3Config()


def load_config(model_path) -> Qwen3Config:
    if isinstance(model_path, Qwen3Config):
        return model_path
    if isinstance(model_path, dict):
        return replace(QWEN3_0_6B, **model_path)
    path = Path(model_path)
    cfg_file = path / "config.json" if path.is_dir() else path
    raw = json.loads(cfg_file.read_text())
    names = {f.name for f in fields(Qwen3Config)}
    kwargs = {k: v for k, v in raw.items() if k in names}
    if "rope_theta" not in kwargs and isinstance(raw.get("rope_parameters"), dict):
        kwargs["rope_theta"] = raw["rope_parameters"].get("rope_theta", QWEN3_0_6B.rope_theta)
    if isinstance(kwargs.get("eos_token_id"), list):
        kwargs["eos_token_id"] = kwargs["eos_token_id"][0]
    if "head_dim" not in kwargs and "hidden_size" in kwargs and "num_attention_heads" in kwargs:
        kwargs["head_dim"] = kwargs["hidden_size"] // kwargs["num_attention_heads"]
    return replace(QWEN3_0_6B, **kwargs)
