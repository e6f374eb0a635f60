"""Writes runner_graphs.json: what the reference's model driver hands its Runner.

Run in the build container only, where /root/reference is mounted:

    python tests/golden/make_runner_fixture.py

The reference's Qwen2 (models/qwen2.py:278-345) calls ``run(graph, inputs,
weights)`` with graphs from build_qwen2, rewritten by quantize.quantize in the
int8 modes. This records, for the seeded tiny model in each mode, each graph's
interface (name, inputs with their shapes, outputs, the weights it reads with
shapes and dtypes), the count of each primitive in it, the attributes of its
int8 matmuls, and the calls one greedy run makes (graph name, token ids, the
past length, output shapes). The fixture is data: nanocompile_amd.runner's
tests rebuild stand-in graphs from it and check HIPBackend recognises them
and follows the same call sequence. Nothing of the reference is copied.
"""

from __future__ import annotations

import json
import os
import sys
from collections import Counter
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REFERENCE = Path(os.environ.get("NANOCOMPILE_REFERENCE", "/root/reference"))
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(REFERENCE))

from nanocompile import interpreter  # noqa: E402  (the reference)
from nanocompile.models.qwen2 import Qwen2, Qwen2Config, greedy  # noqa: E402

from nanocompile_amd.models import config as ours  # noqa: E402  (the seeded weight generator)

PROMPT = [3, 1, 4, 1, 5]


def dims(shape) -> list[str]:
    return [str(d) for d in shape]


def describe(graph) -> dict:
    return {
        "name": graph.name,
        "inputs": [[n.attrs["name"], str(n.dtype), dims(n.shape)] for n in graph.inputs],
        "outputs": {k: [str(v.dtype), dims(v.shape)] for k, v in graph.outputs.items()},
        "weights": {k: [str(v.dtype), dims(v.shape)] for k, v in graph.weights.items()},
        "ops": dict(sorted(Counter(n.op for n in graph.nodes).items())),
        "int8_attrs": sorted({json.dumps(dict(n.attrs), sort_keys=True) for n in graph.nodes
                              if n.op in ("matmul_i8", "matmul_i8_vnni")}),
    }


def main() -> None:
    c = ours.TINY
    config = Qwen2Config(c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
                         c.num_attention_heads, c.num_key_value_heads, c.rms_norm_eps, c.rope_theta,
                         c.tie_word_embeddings)
    weights = ours.random_weights(c, seed=5, std=ours.TINY_STD)
    out = {"prompt": PROMPT, "modes": {}}
    for mode in (None, "int8", "int8-vnni"):
        calls = []

        def run(graph, inputs, w, calls=calls):
            result = interpreter.run(graph, inputs, w)
            calls.append({"graph": graph.name, "token_ids": [int(t) for t in inputs["token_ids"]],
                          "past": int(inputs["past_keys"].shape[2]),
                          "weights": len(w),
                          "outputs": {k: list(v.shape) for k, v in result.items()}})
            return result

        model = Qwen2(config, weights, run=run, quantization=mode)
        tokens = greedy(model, PROMPT, 3)
        out["modes"][mode or "f32"] = {
            "graph": describe(model.graph),
            "graph_last": describe(model.graph_last),
            "weights_passed": sorted(model.weights),
            "calls": calls,
            "tokens": tokens,
        }
    (HERE / "runner_graphs.json").write_text(json.dumps(out, indent=1, sort_keys=True))
    print("wrote runner_graphs.json:", {k: len(v["calls"]) for k, v in out["modes"].items()})


if __name__ == "__main__":
    main()
