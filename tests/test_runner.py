"""HIPBackend recognises the reference's Qwen2 graphs (recorded from the reference itself in
tests/golden/runner_graphs.json) and refuses anything else, before touching a GPU."""

from __future__ import annotations

import copy
import json

import pytest

from tests import runner_graphs


@pytest.fixture(scope="module")
def fixture():
    return runner_graphs.load()


def backend():
    from nanocompile_amd.models.config import TINY
    from nanocompile_amd.runner import HIPBackend
    return HIPBackend(TINY)


@pytest.mark.parametrize("mode", ["f32", "int8", "int8-vnni"])
def test_graphs_are_recognised(fixture, mode):
    b = backend()
    for key, last in (("graph", False), ("graph_last", True)):
        g = runner_graphs.stand_in(fixture["modes"][mode][key])
        assert b.mode(g) == mode
        assert b.last_only(g, mode) is last


@pytest.mark.parametrize("mode", ["f32", "int8", "int8-vnni"])
def test_expected_weights_are_the_references(fixture, mode):
    """The weight names, dtypes and shapes a graph reads, and the names the reference's driver
    passes (quantize.quantized_weights), are exactly what the backend expects."""
    b = backend()
    desc = fixture["modes"][mode]["graph"]
    recorded = {k: (t, tuple(int(d) for d in s)) for k, (t, s) in desc["weights"].items()}
    assert recorded == b.expected_weights(mode)
    assert set(fixture["modes"][mode]["weights_passed"]) == set(b.expected_weights(mode))


def test_the_reference_calls_the_last_row_graph_with_the_cache_so_far(fixture):
    """The protocol the GPU test's driver restates: a prompt, then one token a call."""
    for mode, data in fixture["modes"].items():
        calls = data["calls"]
        prompt = fixture["prompt"]
        assert [c["graph"] for c in calls] == ["qwen2_last"] * 3
        assert calls[0]["token_ids"] == prompt and calls[0]["past"] == 0
        for i, c in enumerate(calls[1:], start=1):
            assert c["token_ids"] == [data["tokens"][i - 1]] and c["past"] == len(prompt) + i - 1
            assert c["outputs"]["logits"] == [1, 256] and c["outputs"]["keys"] == [2, 2, 1, 32]


def test_other_graphs_are_refused(fixture):
    b = backend()
    desc = fixture["modes"]["int8"]["graph"]
    other = copy.deepcopy(desc)
    other["name"] = "mlp"
    with pytest.raises(NotImplementedError, match="Qwen2 forward"):
        b.last_only(runner_graphs.stand_in(other), "int8")
    wider = copy.deepcopy(desc)
    wider["weights"]["model.norm.weight"][1] = ["256"]
    with pytest.raises(NotImplementedError, match="another shape"):
        b.last_only(runner_graphs.stand_in(wider), "int8")
    fewer = copy.deepcopy(desc)
    del fewer["weights"]["model.layers.1.mlp.up_proj.weight@int8"]
    with pytest.raises(NotImplementedError, match="missing"):
        b.last_only(runner_graphs.stand_in(fewer), "int8")
    mixed = copy.deepcopy(desc)
    mixed["ops"]["matmul_i8_vnni"] = 1
    with pytest.raises(NotImplementedError, match="mixes"):
        b.mode(runner_graphs.stand_in(mixed))
    block = copy.deepcopy(fixture["modes"]["int8-vnni"]["graph"])
    block["int8_attrs"] = [json.dumps({"block": 64})]
    with pytest.raises(NotImplementedError, match="block"):
        b.mode(runner_graphs.stand_in(block))


def test_compiled_graph_binds_once_and_checks_bindings(fixture):
    from nanocompile_amd.models.config import TINY
    from nanocompile_amd.runner import HIPBackend, HIPCompiledGraph
    import numpy as np
    b = HIPBackend(TINY)
    g = runner_graphs.stand_in(fixture["modes"]["int8-vnni"]["graph_last"])
    assert b.compiled(g) is b.compiled(g)
    cg = HIPCompiledGraph(g, TINY)
    assert cg.mode == "int8-vnni" and cg.last_only
    inputs = {"token_ids": np.array([1, 2]), "past_keys": np.zeros((2, 2, 3, 32), np.float32),
              "past_values": np.zeros((2, 2, 3, 32), np.float32)}
    with pytest.raises(ValueError, match="disagrees"):
        cg(inputs, {}, bindings={"seq": 3})
    with pytest.raises(NotImplementedError):
        HIPCompiledGraph(runner_graphs.stand_in({**fixture["modes"]["int8"]["graph"], "name": "other"}), TINY)


def test_a_graph_nothing_can_lower_is_refused_with_the_way_out():
    """Without the reference's compiler installed and no lowering given, a graph that is not a
    Qwen2 forward cannot become a program: the error says what to pass."""
    from types import SimpleNamespace

    from nanocompile_amd.runner import HIPCompiledGraph
    with pytest.raises(NotImplementedError, match="program= or lower="):
        HIPCompiledGraph(SimpleNamespace(name="mystery", nodes=[]))


def test_a_cache_view_names_its_host_buffer():
    """The reference hands over ``_keys[:, :, :length]`` (models/qwen2.py:257-258): the backend
    names the sequence by that buffer, whose capacity sizes the device cache. Any other array
    (a fresh one, or a slice that does not start the buffer's rows) names only itself."""
    import numpy as np

    from nanocompile_amd.runner import _owner, _rows_of
    buffer = np.zeros((2, 2, 16, 32), np.float32)
    view = buffer[:, :, :5]
    assert _owner(view) is buffer and _rows_of(buffer, view) == 16
    assert _owner(buffer[:, :, :0]) is buffer
    fresh = np.zeros((2, 2, 5, 32), np.float32)
    assert _owner(fresh) is fresh and _rows_of(fresh, fresh) == 5
    inner = buffer[:, :, 3:8]                      # does not start at the buffer's first row
    assert _owner(inner) is inner and _rows_of(inner, inner) == 5
    heads = buffer[:, :1, :5]                      # a different block shape
    assert _owner(heads) is heads


def test_token_activations_are_an_opt_in_for_the_int8_graphs():
    from nanocompile_amd.models.config import TINY
    from nanocompile_amd.runner import HIPBackend
    assert HIPBackend(TINY).model_quantization("int8") == "int8"
    token = HIPBackend(TINY, activations="token")
    assert [token.model_quantization(m) for m in ("int8", "int8-vnni", "f32")] == ["int8-token", "int8-token", "f32"]
    with pytest.raises(ValueError, match="activations"):
        HIPBackend(TINY, activations="int4")


def test_device_cache_bookkeeping_allocates_once_a_sequence_and_uploads_only_missing_rows(monkeypatch):
    """The Runner's device cache, with the device calls replaced by records: a sequence's first
    call sizes the cache for the host buffer and uploads its filled rows; the calls after it
    allocate nothing and upload nothing the device produced; a new buffer uploads its rows once
    (reusing a cache that is large enough); growth doubles and uploads the rows again; a
    rewound view uploads only rows past what the device still holds."""
    import numpy as np

    from nanocompile_amd import runner
    from nanocompile_amd.models.config import TINY
    made, uploads = [], []

    class FakeCache:
        def __init__(self, capacity):
            self.capacity, self.length, self.keys, self.values = capacity, 0, "k", "v"

    class FakeModel:
        def new_cache(self, capacity):
            made.append(capacity)
            return FakeCache(capacity)

    monkeypatch.setattr(runner, "_upload_rows", lambda device, host, start, stop: uploads.append((device, start, stop)))
    backend = runner.HIPBackend(TINY)
    model = FakeModel()
    shape = (TINY.num_hidden_layers, TINY.num_key_value_heads)

    def buffer(capacity):
        return np.zeros(shape + (capacity, TINY.head_dim), np.float32), np.zeros(shape + (capacity, TINY.head_dim),
                                                                               np.float32)

    def call(kb, vb, past, m):
        seq = backend._cache_for("int8", model, kb[:, :, :past], vb[:, :, :past], past + m)
        seq.held = past + m                    # what run() records after the forward
        return seq

    kb, vb = buffer(19)
    call(kb, vb, 0, 11)
    assert made == [19] and uploads == []
    for past in range(11, 18):
        call(kb, vb, past, 1)
    assert made == [19] and uploads == []
    k2, v2 = buffer(10)                         # another sequence: the cache is large enough
    call(k2, v2, 4, 1)
    assert made == [19] and uploads == [("k", 0, 4), ("v", 0, 4)]
    uploads.clear()
    k3, v3 = buffer(40)                         # a larger buffer: sized for it at once
    call(k3, v3, 30, 1)
    assert made == [19, 40] and uploads == [("k", 0, 30), ("v", 0, 30)]
    uploads.clear()
    k4 = np.zeros(shape + (45, TINY.head_dim), np.float32)   # a view of a fresh array each call: grows
    call(k4, k4.copy(), 44, 1)
    assert made[-1] == 80 and uploads == [("k", 0, 44), ("v", 0, 44)]
    uploads.clear()
    kb, vb = buffer(100)
    call(kb, vb, 0, 20)
    assert made[-1] == 100
    uploads.clear()
    call(kb, vb, 10, 1)                         # rewound to 10: the device still holds 0 .. 9
    assert uploads == []
    call(kb, vb, 15, 1)                         # the caller appended 11 .. 14 itself
    assert uploads == [("k", 11, 15), ("v", 11, 15)]
