"""Qwen2's hyperparameters and seeded random weights in the checkpoint's names.

``Qwen2Config`` carries the fields the reference's ``Qwen2Config`` has
(models/qwen2.py:45-96), with the same validation and the same reading of a
HuggingFace ``config.json``. Weights are named as in the checkpoint
(``model.layers.0.self_attn.q_proj.weight``), as the reference binds them.

There is no network here for real checkpoints: ``random_weights`` draws a
model of the real shape from a seed, in one fixed name order, so every user
(the GPU model, the host oracle, the golden-vector script that runs the
reference) regenerates exactly the same arrays.
"""

from __future__ import annotations

import json
from collections.abc import Iterator, Mapping
from dataclasses import dataclass
from pathlib import Path

import numpy as np


@dataclass(frozen=True)
class Qwen2Config:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    rms_norm_eps: float
    rope_theta: float
    tie_word_embeddings: bool

    def __post_init__(self) -> None:
        if self.hidden_size % self.num_attention_heads:
            raise ValueError("hidden_size must divide evenly into attention heads")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("attention heads must divide evenly into KV heads")
        if self.head_dim % 2:
            raise ValueError("RoPE needs an even head_dim")

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def kv_group_size(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @classmethod
    def from_dict(cls, data: Mapping) -> "Qwen2Config":
        if data.get("architectures") != ["Qwen2ForCausalLM"]:
            raise ValueError(f"not a Qwen2 config: {data.get('architectures')}")
        if data.get("hidden_act", "silu") != "silu":
            raise ValueError(f"hidden_act {data['hidden_act']!r} is not implemented")
        return cls(
            vocab_size=int(data["vocab_size"]),
            hidden_size=int(data["hidden_size"]),
            intermediate_size=int(data["intermediate_size"]),
            num_hidden_layers=int(data["num_hidden_layers"]),
            num_attention_heads=int(data["num_attention_heads"]),
            num_key_value_heads=int(data.get("num_key_value_heads", data["num_attention_heads"])),
            rms_norm_eps=float(data["rms_norm_eps"]),
            rope_theta=float(data.get("rope_theta", 10000.0)),
            tie_word_embeddings=bool(data.get("tie_word_embeddings", False)),
        )

    @classmethod
    def from_model_dir(cls, model_dir: str | Path) -> "Qwen2Config":
        return cls.from_dict(json.loads((Path(model_dir) / "config.json").read_text(encoding="utf-8")))


# Qwen2.5-0.5B's shape, and a tiny one for tests.
QWEN25_05B = Qwen2Config(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_hidden_layers=24,
                         num_attention_heads=14, num_key_value_heads=2, rms_norm_eps=1e-6, rope_theta=1e6,
                         tie_word_embeddings=True)
TINY_STD = 0.15            # the weight scale tests draw TINY's weights at
TINY = Qwen2Config(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                   num_attention_heads=4, num_key_value_heads=2, rms_norm_eps=1e-6, rope_theta=1e6,
                   tie_word_embeddings=True)

PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def weight_shapes(config: Qwen2Config) -> Iterator[tuple[str, tuple[int, ...]]]:
    """Every weight of the model, in the one order ``random_weights`` draws them."""
    h, inter, d = config.hidden_size, config.intermediate_size, config.head_dim
    q_out, kv_out = config.num_attention_heads * d, config.num_key_value_heads * d
    yield "model.embed_tokens.weight", (config.vocab_size, h)
    for i in range(config.num_hidden_layers):
        p = f"model.layers.{i}"
        yield f"{p}.input_layernorm.weight", (h,)
        yield f"{p}.self_attn.q_proj.weight", (q_out, h)
        yield f"{p}.self_attn.q_proj.bias", (q_out,)
        yield f"{p}.self_attn.k_proj.weight", (kv_out, h)
        yield f"{p}.self_attn.k_proj.bias", (kv_out,)
        yield f"{p}.self_attn.v_proj.weight", (kv_out, h)
        yield f"{p}.self_attn.v_proj.bias", (kv_out,)
        yield f"{p}.self_attn.o_proj.weight", (h, q_out)
        yield f"{p}.post_attention_layernorm.weight", (h,)
        yield f"{p}.mlp.gate_proj.weight", (inter, h)
        yield f"{p}.mlp.up_proj.weight", (inter, h)
        yield f"{p}.mlp.down_proj.weight", (h, inter)
    yield "model.norm.weight", (h,)
    if not config.tie_word_embeddings:
        yield "lm_head.weight", (config.vocab_size, h)


def random_weights(config: Qwen2Config, seed: int = 0, std: float = 0.02) -> dict[str, np.ndarray]:
    """Seeded random-init weights: N(0, std) matrices and biases, norms 1 + N(0, 0.1).

    ``std`` defaults to BASELINE's 0.02. Tiny test models use a larger one: at
    0.02 a 128-wide model's layers barely move the residual stream and greedy
    decoding repeats its input token, which would make token checks vacuous.
    """
    rng = np.random.default_rng(seed)
    out: dict[str, np.ndarray] = {}
    for name, shape in weight_shapes(config):
        if name.endswith("layernorm.weight") or name == "model.norm.weight":
            out[name] = (1.0 + 0.1 * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
        else:
            out[name] = (np.float32(std) * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
    return out
