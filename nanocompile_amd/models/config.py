"""Qwen2's hyperparameters and seeded random weights in the checkpoint's names.

A model is described by nine numbers; their names are the ones HuggingFace's
``config.json`` uses and the reference's model driver reads
(models/qwen2.py:45-96), so a configuration object from either side can be
handed to this package (``Qwen2Config.coerce`` accepts any object that has
them). What this package needs of them is checked by ``problems``: the
kernels assume the head width splits the hidden width, the query heads split
evenly over the KV heads, and RoPE's half-split pairing needs an even head
width.

Weights are named as in the checkpoint
(``model.layers.0.self_attn.q_proj.weight``). There is no network here for
real checkpoints: ``random_weights`` draws a model of the real shape from a
seed, in one fixed name order, so every user (the GPU model, the host oracle,
the golden-vector script that runs the reference) regenerates exactly the
same arrays.
"""

from __future__ import annotations

import json
from collections.abc import Iterator, Mapping
from dataclasses import dataclass, fields
from pathlib import Path

import numpy as np

# config.json key -> (field, type, value when the key is absent; None = required)
_JSON_KEYS = {
    "vocab_size": ("vocab_size", int, None),
    "hidden_size": ("hidden_size", int, None),
    "intermediate_size": ("intermediate_size", int, None),
    "num_hidden_layers": ("num_hidden_layers", int, None),
    "num_attention_heads": ("num_attention_heads", int, None),
    "num_key_value_heads": ("num_key_value_heads", int, "num_attention_heads"),
    "rms_norm_eps": ("rms_norm_eps", float, None),
    "rope_theta": ("rope_theta", float, 10000.0),
    "tie_word_embeddings": ("tie_word_embeddings", bool, False),
}


@dataclass(frozen=True)
class Qwen2Config:
    """The nine hyperparameters of a Qwen2 decoder (HuggingFace's names)."""

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
        found = self.problems()
        if found:
            raise ValueError(f"unusable Qwen2 configuration: {'; '.join(found)}")

    def problems(self) -> list[str]:
        """What in this configuration the kernels cannot run, as sentences (empty when fine)."""
        out = []
        sizes = {f.name: getattr(self, f.name) for f in fields(self) if f.type in ("int", int)}
        out += [f"{name} = {value} is not positive" for name, value in sizes.items() if value <= 0]
        if out:
            return out
        heads, kv = self.num_attention_heads, self.num_key_value_heads
        if self.hidden_size % heads:
            out.append(f"{heads} query heads do not split hidden_size {self.hidden_size}")
        elif (self.hidden_size // heads) % 2:
            out.append(f"head width {self.hidden_size // heads} is odd; RoPE pairs its halves")
        if heads % kv:
            out.append(f"{heads} query heads do not share {kv} KV heads evenly")
        return out

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def queries_per_kv(self) -> int:
        """Query heads reading each KV head (head h reads KV head h // this)."""
        return self.num_attention_heads // self.num_key_value_heads

    @classmethod
    def coerce(cls, config) -> "Qwen2Config":
        """This package's config from any object with the nine fields (the reference's included)."""
        if isinstance(config, cls):
            return config
        missing = [f.name for f in fields(cls) if not hasattr(config, f.name)]
        if missing:
            raise TypeError(f"{type(config).__name__} lacks Qwen2 fields {missing}")
        return cls(**{f.name: getattr(config, f.name) for f in fields(cls)})

    @classmethod
    def from_json(cls, source: str | Path | Mapping) -> "Qwen2Config":
        """From a HuggingFace ``config.json``: a mapping, the file, or the model directory holding it."""
        if isinstance(source, Mapping):
            data = source
        else:
            path = Path(source)
            data = json.loads((path / "config.json" if path.is_dir() else path).read_text(encoding="utf-8"))
        arch = data.get("architectures") or []
        if "Qwen2ForCausalLM" not in arch or data.get("hidden_act", "silu") != "silu":
            raise ValueError(f"config.json describes {arch} with activation {data.get('hidden_act')!r}; "
                             f"this package runs Qwen2ForCausalLM with SiLU")
        values = {}
        for key, (name, kind, default) in _JSON_KEYS.items():
            if key in data:
                values[name] = kind(data[key])
            elif default is None:
                raise ValueError(f"config.json has no {key!r}")
            else:
                values[name] = kind(data[default]) if isinstance(default, str) else default
        return cls(**values)

    from_model_dir = from_json


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
