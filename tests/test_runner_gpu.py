"""The reference's model driver on HIPBackend: greedy tokens and logits of the reference's compiled C.

The driver below restates the reference's Qwen2.forward / greedy (models/qwen2.py:316-368: the
last-row graph for generation, the host cache's filled part passed each call, the new keys and
values appended after) over stand-ins of the reference's own graphs (tests/golden/
runner_graphs.json). Its call sequence must be the one the reference made when the fixture was
recorded; its tokens and logits must be golden G5's (the reference's Qwen2 on its C backend).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import reference as R
from tests import runner_graphs

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
PROMPTS = ([4, 5, 6], [7, 8], [1], [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5])     # make_golden.py's G5 prompts
TAGS = {"f32": "f32", "int8": "int8", "int8-vnni": "vnni"}


class HostCache:
    """The reference's KVCache contents (models/qwen2.py:232-271), grown by concatenation."""

    def __init__(self, config) -> None:
        shape = (config.num_hidden_layers, config.num_key_value_heads, 0, config.head_dim)
        self.keys, self.values = np.zeros(shape, np.float32), np.zeros(shape, np.float32)

    def append(self, keys, values) -> None:
        self.keys = np.concatenate([self.keys, keys], axis=2)
        self.values = np.concatenate([self.values, values], axis=2)


class ReferenceCache:
    """The reference's KVCache as its driver uses it (models/qwen2.py:232-271): one preallocated
    buffer per side, grown by doubling; each call is handed a view of the filled rows."""

    def __init__(self, config, capacity: int) -> None:
        self.config, self.length = config, 0
        self._keys, self._values = self._allocate(capacity), self._allocate(capacity)

    def _allocate(self, capacity: int) -> np.ndarray:
        c = self.config
        return np.zeros((c.num_hidden_layers, c.num_key_value_heads, capacity, c.head_dim), np.float32)

    @property
    def keys(self) -> np.ndarray:
        return self._keys[:, :, :self.length]

    @property
    def values(self) -> np.ndarray:
        return self._values[:, :, :self.length]

    def append(self, keys, values) -> None:
        n = keys.shape[2]
        if self.length + n > self._keys.shape[2]:
            capacity = max(self.length + n, 2 * self._keys.shape[2])
            for name in ("_keys", "_values"):
                grown = self._allocate(capacity)
                grown[:, :, :self.length] = getattr(self, name)[:, :, :self.length]
                setattr(self, name, grown)
        self._keys[:, :, self.length:self.length + n] = keys
        self._values[:, :, self.length:self.length + n] = values
        self.length += n


class Driver:
    """models/qwen2.py:316-368 over a Runner, recording each call."""

    def __init__(self, config, run, graphs, weights) -> None:
        self.config, self.run, self.graphs, self.weights, self.calls = config, run, graphs, weights, []

    def forward(self, ids, cache=None, last_only=False):
        ids = np.asarray(ids, np.int64)
        if cache is None:
            cache = HostCache(self.config)
            keep = False
        else:
            keep = True
        graph = self.graphs["graph_last" if last_only else "graph"]
        out = self.run(graph, {"token_ids": ids, "past_keys": cache.keys, "past_values": cache.values},
                       self.weights)
        self.calls.append({"graph": graph.name, "token_ids": [int(t) for t in ids],
                           "past": int(cache.keys.shape[2]),
                           "outputs": {k: list(v.shape) for k, v in out.items()}})
        if keep:
            cache.append(out["keys"], out["values"])
        return out["logits"]

    def greedy(self, prompt, n, cache=None):
        cache = HostCache(self.config) if cache is None else cache
        pending, out = list(prompt), []
        for _ in range(n):
            token = int(np.argmax(self.forward(pending, cache, last_only=True)[0]))
            out.append(token)
            pending = [token]
        return out


@pytest.fixture(scope="module")
def setup(gpu):
    from nanocompile_amd.models.config import TINY, random_weights
    from nanocompile_amd.runner import HIPBackend
    meta = json.loads((GOLDEN / "golden.json").read_text())["g5"]
    weights = random_weights(TINY, seed=meta["seed"], std=meta["std"])
    quantized = dict(weights)
    for name in list(weights):                       # quantize.quantized_weights' names
        if name.endswith("_proj.weight"):
            q, s = R.quantize_int8(weights[name])
            quantized[f"{name}@int8"], quantized[f"{name}@scales"] = q, s
    fixture = runner_graphs.load()
    golden = np.load(GOLDEN / "golden.npz", allow_pickle=False)
    return TINY, HIPBackend(TINY, max_tokens=64), weights, quantized, fixture, golden


def driver(setup, mode):
    config, backend, weights, quantized, fixture, _ = setup
    graphs = {k: runner_graphs.stand_in(fixture["modes"][mode][k]) for k in ("graph", "graph_last")}
    passed = {n: (weights if mode == "f32" else quantized)[n] for n in fixture["modes"][mode]["weights_passed"]}
    return Driver(config, backend, graphs, passed)


@pytest.mark.parametrize("mode", ["f32", "int8", "int8-vnni"])
def test_greedy_through_the_runner_is_the_references(setup, mode):
    golden = setup[5]
    print(f"runner greedy {mode}", flush=True)
    d = driver(setup, mode)
    for i, prompt in enumerate(PROMPTS):
        assert d.greedy(prompt, 8) == [int(t) for t in golden[f"g5_{TAGS[mode]}_tokens_{i}"]], (mode, i)


@pytest.mark.parametrize("mode", ["f32", "int8", "int8-vnni"])
def test_call_sequence_is_the_references(setup, mode):
    fixture = setup[4]
    d = driver(setup, mode)
    tokens = d.greedy(fixture["prompt"], 3)
    assert tokens == fixture["modes"][mode]["tokens"]
    assert d.calls == [{k: c[k] for k in ("graph", "token_ids", "past", "outputs")}
                       for c in fixture["modes"][mode]["calls"]]


@pytest.mark.parametrize("mode", ["f32", "int8", "int8-vnni"])
def test_logits_keys_and_values_through_the_runner(setup, mode):
    config, golden = setup[0], setup[5]
    d = driver(setup, mode)
    ids = np.array(PROMPTS[3])
    logits = d.forward(ids)                                  # the full graph, no cache
    ref = golden[f"g5_{TAGS[mode]}_logits"]
    assert logits.shape == ref.shape
    assert np.max(np.abs(logits - ref)) / np.max(np.abs(ref)) <= 1e-4
    cache = HostCache(config)
    d.forward(ids[:6], cache)
    step = d.forward(ids[6:7], cache, last_only=True)
    ref = golden[f"g5_{TAGS[mode]}_decode_logits"]
    assert np.max(np.abs(step - ref)) / np.max(np.abs(ref)) <= 1e-4
    assert cache.keys.shape == (config.num_hidden_layers, config.num_key_value_heads, 7, config.head_dim)
    assert np.isfinite(cache.keys).all() and np.isfinite(cache.values).all()


@pytest.mark.parametrize("mode", ["int8", "int8-vnni", "f32"])
def test_the_references_cache_is_held_on_the_device_and_nothing_is_allocated_after_the_first_call(setup, mode):
    """With the reference's own cache (one buffer sized for the sequence, views of its filled
    rows), the first call allocates the device cache and every later call of the sequence
    allocates nothing, uploading none of the rows the device produced; the tokens are G5's."""
    from nanocompile_amd import hip
    config, golden = setup[0], setup[5]
    d = driver(setup, mode)
    for i, prompt in enumerate(PROMPTS):
        cache = ReferenceCache(config, len(prompt) + 8)
        first = d.forward(prompt, cache, last_only=True)
        before = hip.allocations()
        tokens = [int(np.argmax(first[0]))]
        for _ in range(7):
            tokens.append(int(np.argmax(d.forward([tokens[-1]], cache, last_only=True)[0])))
        assert hip.allocations() == before, (mode, i)
        assert tokens == [int(t) for t in golden[f"g5_{TAGS[mode]}_tokens_{i}"]], (mode, i)


def test_a_growing_or_rewound_host_cache_gives_the_same_results(setup):
    """A cache that starts too small and doubles (each growth a new host buffer, uploaded once),
    and a cache rewound and refilled with other tokens (the device's rows past the new length
    no longer count): the same logits as a fresh run."""
    config, golden = setup[0], setup[5]
    d = driver(setup, "int8")
    prompt = PROMPTS[3]
    grown = ReferenceCache(config, 2)
    assert d.greedy(prompt, 8, cache=grown) == [int(t) for t in golden["g5_int8_tokens_3"]]
    assert grown._keys.shape[2] >= len(prompt) + 7
    ids = np.array(PROMPTS[3])
    cache = ReferenceCache(config, 16)
    d.forward(ids[:6], cache)
    d.forward(ids[6:9], cache)
    cache.length = 6                          # rewind: rows 6.. are refilled with other tokens
    d.forward(ids[8:9], cache)
    step = d.forward(ids[6:7], cache, last_only=True)
    fresh = ReferenceCache(config, 16)
    d.forward(ids[:6], fresh)
    d.forward(ids[8:9], fresh)
    want = d.forward(ids[6:7], fresh, last_only=True)
    assert np.array_equal(step.view(np.uint32), want.view(np.uint32))


def test_token_activations_through_the_runner_are_the_per_token_model(setup):
    """``HIPBackend(config, activations="token")`` runs the reference's int8 graphs on the
    per-token model: its greedy tokens and logits are Qwen2(..., "int8-token")'s, bit for bit."""
    from nanocompile_amd.models.qwen2 import Qwen2, greedy
    from nanocompile_amd.runner import HIPBackend
    config, _, _, quantized, fixture, _ = setup
    backend = HIPBackend(config, max_tokens=64, activations="token")
    for mode in ("int8", "int8-vnni"):
        graphs = {k: runner_graphs.stand_in(fixture["modes"][mode][k]) for k in ("graph", "graph_last")}
        passed = {n: quantized[n] for n in fixture["modes"][mode]["weights_passed"]}
        d = Driver(config, backend, graphs, passed)
        model = Qwen2(config, passed, quantization="int8-token", max_tokens=64)
        for prompt in PROMPTS:
            want = greedy(model, prompt, 8)
            assert d.greedy(prompt, 8, cache=ReferenceCache(config, len(prompt) + 8)) == want, (mode, prompt)
            assert model.generate(prompt, 8) == want
        ids = np.array(PROMPTS[3])
        got = d.forward(ids, ReferenceCache(config, 16), last_only=True)
        want = model.forward(ids, model.new_cache(16), last_only=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), mode
