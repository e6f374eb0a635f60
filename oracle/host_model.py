"""The host C Qwen2 (oracle/nc_model.c): the GPU model's bit-level oracle and the CPU baseline.

TEST INFRASTRUCTURE ONLY. Weights are quantized here with the NumPy
restatement of the reference's quantizer (reference.quantize_int8), the three
attention projections concatenated row-wise (q, then k, then v: per-row
quantization makes that exact), and the LM head table laid out in blocks of
8 rows for the host's vector loop (each row still summed in k order).
"""

from __future__ import annotations

import ctypes

import numpy as np

from oracle import host
from oracle import reference as R

_P, _I, _F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float


class LayerW(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("gamma1", "gamma2", "qkv_q", "qkv_s", "qkv_b", "o_q", "o_s", "g_q", "u_q",
                                  "g_s", "u_s", "d_q", "d_s")]


class ModelT(ctypes.Structure):
    _fields_ = [("vocab", _I), ("hidden", _I), ("inter", _I), ("layers", _I), ("heads", _I), ("kv", _I),
                ("d", _I), ("capacity", _I), ("eps", _F), ("scale", _F), ("embed", _P), ("table8", _P),
                ("norm", _P), ("inv_freq", _P), ("w", ctypes.POINTER(LayerW)), ("kcache", _P), ("vcache", _P)]


def inverse_frequencies(head_dim: int, theta: float) -> np.ndarray:
    """RoPE rates exactly as the reference computes them (nn.py:69-75)."""
    exponent = np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / np.float32(head_dim)
    return (np.float32(1.0) / (np.float32(theta) ** exponent)).astype(np.float32)


def _c(a):
    return a.ctypes.data


class HostQwen2:
    """Qwen2 with int8 projections and per-token int8 activations, in host C."""

    def __init__(self, config, weights, capacity: int = 1024) -> None:
        lib = host.load()
        lib.nc_host_qwen2_forward.argtypes = [_P, _P, _I, _I, _P, ctypes.c_int]
        lib.nc_host_qwen2_forward.restype = _I
        lib.nc_host_model_struct_size.restype = _I
        lib.nc_host_layer_struct_size.restype = _I
        assert lib.nc_host_model_struct_size() == ctypes.sizeof(ModelT)
        assert lib.nc_host_layer_struct_size() == ctypes.sizeof(LayerW)
        self.lib, self.config, self.capacity = lib, config, capacity
        c = config
        self._keep: list[np.ndarray] = []

        def keep(a):
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return _c(a)

        layers = (LayerW * c.num_hidden_layers)()
        for i in range(c.num_hidden_layers):
            p = f"model.layers.{i}"
            qkv = [R.quantize_int8(weights[f"{p}.self_attn.{n}_proj.weight"]) for n in "qkv"]
            q8 = {n: R.quantize_int8(weights[f"{p}.mlp.{n}_proj.weight"]) for n in ("gate", "up", "down")}
            o8 = R.quantize_int8(weights[f"{p}.self_attn.o_proj.weight"])
            layers[i] = LayerW(
                keep(weights[f"{p}.input_layernorm.weight"]), keep(weights[f"{p}.post_attention_layernorm.weight"]),
                keep(np.concatenate([v for v, _ in qkv])), keep(np.concatenate([s for _, s in qkv])),
                keep(np.concatenate([weights[f"{p}.self_attn.{n}_proj.bias"] for n in "qkv"])),
                keep(o8[0]), keep(o8[1]), keep(q8["gate"][0]), keep(q8["up"][0]), keep(q8["gate"][1]),
                keep(q8["up"][1]), keep(q8["down"][0]), keep(q8["down"][1]))
        self._layers = layers
        embed = np.ascontiguousarray(weights["model.embed_tokens.weight"], np.float32)
        head = embed if c.tie_word_embeddings else np.ascontiguousarray(weights["lm_head.weight"], np.float32)
        v, h = head.shape
        blocks = -(-v // 8)
        padded = np.zeros((blocks * 8, h), np.float32)
        padded[:v] = head
        table8 = padded.reshape(blocks, 8, h).transpose(0, 2, 1).copy()
        shape = (c.num_hidden_layers, c.num_key_value_heads, capacity, c.head_dim)
        self.kcache, self.vcache = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
        self.model = ModelT(c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
                            c.num_attention_heads, c.num_key_value_heads, c.head_dim, capacity,
                            np.float32(c.rms_norm_eps), np.float32(c.head_dim ** -0.5),
                            keep(embed), keep(table8), keep(weights["model.norm.weight"]),
                            keep(inverse_frequencies(c.head_dim, c.rope_theta)), layers,
                            _c(self.kcache), _c(self.vcache))
        self.length = 0

    def reset(self) -> None:
        self.length = 0

    def forward(self, ids, all_rows: bool = False) -> tuple[np.ndarray, int]:
        """Logits of the new tokens (the last row, or all) and the last row's argmax; advances the cache."""
        ids = np.ascontiguousarray(ids, np.int64)
        rows = len(ids) if all_rows else 1
        logits = np.empty((rows, self.config.vocab_size), np.float32)
        token = self.lib.nc_host_qwen2_forward(ctypes.byref(self.model), _c(ids), len(ids), self.length,
                                               _c(logits), int(all_rows))
        if token == -1:
            raise ValueError("a token id is outside the vocabulary")
        if token == -2:
            raise ValueError("the cache is full")
        self.length += len(ids)
        return logits, int(token)

    def greedy(self, prompt, max_new_tokens: int) -> list[int]:
        """The reference's greedy (models/qwen2.py:348-368) with a cache."""
        self.reset()
        out: list[int] = []
        pending = list(prompt)
        for _ in range(max_new_tokens):
            _, token = self.forward(pending)
            out.append(token)
            pending = [token]
        return out
