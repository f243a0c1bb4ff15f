"""Llama model shapes (the fields of the reference's ModelConfig, src/kvserve/config.py:24-75)."""

from __future__ import annotations

import json
from dataclasses import asdict, dataclass, replace
from pathlib import Path


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_scaling: dict | None = None
    max_position_embeddings: int = 131072
    tie_word_embeddings: bool = False

    @classmethod
    def from_dir(cls, path: Path) -> ModelConfig:
        """From a Hugging Face config.json (model_type llama)."""
        cfg = json.loads((Path(path) / "config.json").read_text())
        if cfg.get("model_type") != "llama":
            raise ValueError(f"unsupported model_type {cfg.get('model_type')!r}; only llama is supported")
        heads = cfg["num_attention_heads"]
        rope_theta = cfg.get("rope_theta", 10000.0)
        rope_scaling = cfg.get("rope_scaling")
        if "rope_parameters" in cfg:  # transformers >= 5 writes one merged dictionary
            rp = dict(cfg["rope_parameters"] or {})
            rope_theta = rp.pop("rope_theta", rope_theta)
            rope_scaling = rp if rp.get("rope_type", "default") != "default" else None
        return cls(
            vocab_size=cfg["vocab_size"],
            hidden_size=cfg["hidden_size"],
            intermediate_size=cfg["intermediate_size"],
            num_layers=cfg["num_hidden_layers"],
            num_heads=heads,
            num_kv_heads=cfg.get("num_key_value_heads", heads),
            head_dim=cfg.get("head_dim") or cfg["hidden_size"] // heads,
            rms_norm_eps=cfg["rms_norm_eps"],
            rope_theta=rope_theta,
            rope_scaling=rope_scaling,
            max_position_embeddings=cfg["max_position_embeddings"],
            tie_word_embeddings=cfg.get("tie_word_embeddings", False),
        )

    def to_hf_dict(self) -> dict:
        """A Hugging Face style config.json for this shape."""
        d = {
            "model_type": "llama",
            "architectures": ["LlamaForCausalLM"],
            "vocab_size": self.vocab_size,
            "hidden_size": self.hidden_size,
            "intermediate_size": self.intermediate_size,
            "num_hidden_layers": self.num_layers,
            "num_attention_heads": self.num_heads,
            "num_key_value_heads": self.num_kv_heads,
            "head_dim": self.head_dim,
            "rms_norm_eps": self.rms_norm_eps,
            "rope_theta": self.rope_theta,
            "max_position_embeddings": self.max_position_embeddings,
            "tie_word_embeddings": self.tie_word_embeddings,
            "hidden_act": "silu",
            "attention_bias": False,
            "mlp_bias": False,
        }
        if self.rope_scaling is not None:
            d["rope_scaling"] = dict(self.rope_scaling)
        return d

    def with_layers(self, n: int) -> ModelConfig:
        return replace(self, num_layers=n)

    def as_dict(self) -> dict:
        return asdict(self)


_LLAMA3_ROPE = {
    "rope_type": "llama3",
    "factor": 32.0,
    "low_freq_factor": 1.0,
    "high_freq_factor": 4.0,
    "original_max_position_embeddings": 8192,
}

# Published shapes of the two models the reference's numbers are quoted on.
LLAMA_3_2_1B = ModelConfig(
    vocab_size=128256, hidden_size=2048, intermediate_size=8192, num_layers=16, num_heads=32, num_kv_heads=8,
    head_dim=64, rms_norm_eps=1e-5, rope_theta=500000.0, rope_scaling=_LLAMA3_ROPE,
    max_position_embeddings=131072, tie_word_embeddings=True,
)  # fmt: skip
LLAMA_3_1_8B = ModelConfig(
    vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_layers=32, num_heads=32, num_kv_heads=8,
    head_dim=128, rms_norm_eps=1e-5, rope_theta=500000.0, rope_scaling={**_LLAMA3_ROPE, "factor": 8.0},
    max_position_embeddings=131072, tie_word_embeddings=False,
)  # fmt: skip
