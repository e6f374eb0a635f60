"""The reference's ``Runner`` on the GPU: ``HIPBackend(config)(graph, inputs, weights) -> dict``.

The reference's model driver runs every step as ``run(graph, inputs, weights)``
(models/qwen2.py:229 declares the protocol, 337-342 calls it): ``graph`` is the
forward pass from ``build_qwen2`` (models/qwen2.py:167-224), rewritten by
``quantize.quantize`` in the int8 modes (quantize.py:127-164); ``inputs`` are
``token_ids`` and the host cache's filled part, ``past_keys`` and
``past_values`` ``[layers, kv_heads, past, head_dim]``; ``weights`` are what the
graph reads (``quantize.quantized_weights``, quantize.py:167-180: ``W@int8``
and ``W@scales`` for each int8 projection, float32 for the rest). It returns
``logits`` (``[seq, vocab]``, or ``[1, vocab]`` for ``qwen2_last``) and the
new tokens' ``keys`` and ``values`` ``[layers, kv_heads, seq, head_dim]`` as
host arrays, as the reference's compiled runtime does (runtime.py:245-301).

``HIPBackend`` is that callable for these graphs, so the reference's own
``Qwen2(config, weights, run=HIPBackend(config), quantization=...)`` and its
``greedy`` run their steps on this package's kernels. It recognises a graph
by its interface (names, inputs, outputs, the weights it reads and their
shapes) and by its int8 primitive (``matmul_i8``: the reference's "int8" mode,
``matmul_i8_vnni`` with block 32: "int8-vnni", neither: float32), and runs the
GPU model in the same mode, whose kernels compute the reference's kernels'
bits (the int8 and float32 projections) or its operations in a stated order
(rms_norm, softmax, attention). Any other graph runs as generated HIP: the
reference's compiled program for it, lowered by codegen_hip with GPU
schedules and run from one device arena (compiled.py), the reference's own
kernels' arithmetic in the reference's order.

On the model path the model, with its weights uploaded and packed, is made
once per mode and kept for the weights mapping it was last called with. The
reference keeps its cache on the host and hands the filled part over every
call, a view of one buffer that its KVCache grows by doubling
(models/qwen2.py:232-271); the backend keeps one device cache per mode for
the sequence it was last called with, identified by the host buffer those
views come from. The rows the device produced itself (the keys and values it
returned, which the caller appends at the rows after ``past``) are not
uploaded again: a call uploads only the rows the device does not hold, and
downloads only the new rows. A new buffer (another sequence, or the host
cache grown into a fresh buffer) uploads its filled part once. The device
cache is allocated when a sequence needs more rows than it has, sized to the
host buffer's capacity, so a sequence whose host cache is made for its whole
length (as the reference's ``greedy`` makes it) allocates nothing after its
first call. Rows are trusted by position, as weights are by identity: a
caller that rewrites rows of its cache in place, rather than appending, must
hand over a fresh buffer (or call ``forget``).

``activations="token"`` is an opt-in numeric deviation: graphs the reference
built in its ``int8`` or ``int8-vnni`` mode run on the per-token model
(``quantization="int8-token"``: the same per-row int8 weights, each token's
activations quantized with one scale, exact int32 accumulation), which is
this package's fast decode path. Its logits differ from the reference mode's
by the activations' quantization error; its tokens are the per-token model's.
``HIPCompiledGraph`` is the per-graph form, the reference's
``CompiledGraph(graph, ...)(inputs, weights, bindings, profile)``
(runtime.py:167-301), which ``HIPBackend.compiled`` makes once per graph as
the reference's ``CBackend.compiled`` does (runtime.py:321-333).
"""

from __future__ import annotations

import time
from collections.abc import Mapping

import numpy as np

from nanocompile_amd.models.config import Qwen2Config

INPUTS = ("token_ids", "past_keys", "past_values")
OUTPUTS = {"logits", "keys", "values"}
INT8_OPS = {"matmul_i8": "int8", "matmul_i8_vnni": "int8-vnni"}
VNNI_BLOCK = 32
PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


class HIPBackend:
    """A ``Runner`` (models/qwen2.py:229) on the GPU: ``run(graph, inputs, weights) -> dict``.

    Each graph is compiled once, on first use (the reference's CBackend, runtime.py:321-337), by
    :class:`HIPCompiledGraph`: Qwen2 forward graphs of ``config`` (the reference's ``Qwen2Config``
    or this package's: the same fields) on the model library, every other graph as generated HIP.
    ``max_tokens`` bounds one call's tokens on the model path; ``schedule``, ``fuse`` and ``lower``
    are passed to each HIPCompiledGraph.
    """

    def __init__(self, config=None, max_tokens: int = 512, device: int = 0, schedule="default",
                 fuse: bool = True, lower=None, activations: str = "reference") -> None:
        if activations not in ("reference", "token"):
            raise ValueError("activations must be 'reference' (the graph's own int8 mode) or 'token' "
                             "(per-token int8 activations, a numeric deviation)")
        self.config = None if config is None else Qwen2Config.coerce(config)
        self.max_tokens, self.device, self.schedule = max_tokens, device, schedule
        self.fuse, self.lower, self.activations = fuse, lower, activations
        # one model per mode, for the weights mapping it was last called with: a new
        # mapping replaces (and frees) the model made for the old one
        self._models: dict[str, tuple[Mapping, object]] = {}
        # one device cache per mode, for the sequence last run in it
        self._sequences: dict[str, _Sequence] = {}
        self._compiled: list[tuple[object, "HIPCompiledGraph"]] = []

    # -- recognising a graph ----------------------------------------------------------------

    def mode(self, graph) -> str:
        """The quantization mode a Qwen2 graph was built in: "f32", "int8" or "int8-vnni"."""
        found = {INT8_OPS[node.op] for node in graph.nodes if node.op in INT8_OPS}
        if len(found) > 1:
            raise NotImplementedError(f"graph {graph.name!r} mixes matmul_i8 and matmul_i8_vnni")
        mode = found.pop() if found else "f32"
        if mode == "int8-vnni":
            blocks = {node.attrs["block"] for node in graph.nodes if node.op == "matmul_i8_vnni"}
            if blocks != {VNNI_BLOCK}:
                raise NotImplementedError(f"matmul_i8_vnni with block {sorted(blocks)}; this backend "
                                          f"runs block {VNNI_BLOCK} (quantize.py:44)")
        return mode

    def expected_weights(self, mode: str) -> dict[str, tuple[str, tuple[int, ...]]]:
        """The weights a Qwen2 graph of this configuration reads in ``mode``: name -> (dtype, shape)."""
        c = self.config
        h, inter, d = c.hidden_size, c.intermediate_size, c.head_dim
        q_out, kv_out = c.num_attention_heads * d, c.num_key_value_heads * d
        out: dict[str, tuple[str, tuple[int, ...]]] = {"model.embed_tokens.weight": ("f32", (c.vocab_size, h)),
                                                       "model.norm.weight": ("f32", (h,))}
        if not c.tie_word_embeddings:
            out["lm_head.weight"] = ("f32", (c.vocab_size, h))
        shapes = {"self_attn.q_proj": (q_out, h), "self_attn.k_proj": (kv_out, h),
                  "self_attn.v_proj": (kv_out, h), "self_attn.o_proj": (h, q_out),
                  "mlp.gate_proj": (inter, h), "mlp.up_proj": (inter, h), "mlp.down_proj": (h, inter)}
        for layer in range(c.num_hidden_layers):
            p = f"model.layers.{layer}"
            out[f"{p}.input_layernorm.weight"] = ("f32", (h,))
            out[f"{p}.post_attention_layernorm.weight"] = ("f32", (h,))
            for name in ("q_proj", "k_proj", "v_proj"):
                out[f"{p}.self_attn.{name}.bias"] = ("f32", (shapes[f"self_attn.{name}"][0],))
            for proj in PROJECTIONS:
                w = f"{p}.{proj}.weight"
                if mode == "f32":
                    out[w] = ("f32", shapes[proj])
                else:
                    out[f"{w}@int8"] = ("i8", shapes[proj])
                    out[f"{w}@scales"] = ("f32", (shapes[proj][0],))
        return out

    def last_only(self, graph, mode: str) -> bool:
        """Check ``graph`` is a Qwen2 forward of this configuration; True for the last-row variant."""
        if self.config is None:
            raise NotImplementedError("no Qwen2 configuration given: every graph runs as generated code")
        if graph.name not in ("qwen2", "qwen2_last"):
            raise NotImplementedError(f"graph {graph.name!r}: this backend runs the Qwen2 forward graphs "
                                      f"(models/qwen2.py:167-224), 'qwen2' and 'qwen2_last'")
        names = tuple(node.attrs["name"] for node in graph.inputs)
        if names != INPUTS or set(graph.outputs) != OUTPUTS:
            raise NotImplementedError(f"graph {graph.name!r} has inputs {names} and outputs "
                                      f"{sorted(graph.outputs)}, not a Qwen2 forward's")
        expected = self.expected_weights(mode)
        reads = {name: (str(node.dtype), tuple(int(str(d)) for d in node.shape))
                 for name, node in graph.weights.items()}
        if reads != expected:
            missing, extra = sorted(set(expected) - set(reads)), sorted(set(reads) - set(expected))
            wrong = sorted(n for n in set(reads) & set(expected) if reads[n] != expected[n])
            raise NotImplementedError(f"graph {graph.name!r} is not this configuration's Qwen2 in mode "
                                      f"{mode!r}: weights missing {missing[:3]}, unexpected {extra[:3]}, "
                                      f"of another shape {wrong[:3]}")
        return graph.name == "qwen2_last"

    # -- running it -----------------------------------------------------------------------------

    def model_quantization(self, mode: str) -> str:
        """The GPU model's quantization for a graph of ``mode``: the mode itself, or with
        ``activations="token"`` the per-token model for either int8 mode."""
        if self.activations == "token" and mode in ("int8", "int8-vnni"):
            return "int8-token"
        return mode

    def _model(self, mode: str, weights: Mapping):
        held = self._models.get(mode)
        if held is not None and held[0] is weights:
            return held[1]
        self._models.pop(mode, None)          # drop the old weights' device arena before uploading new ones
        self._sequences.pop(mode, None)
        from nanocompile_amd.models.qwen2 import Qwen2
        model = Qwen2(self.config, weights, quantization=self.model_quantization(mode), max_tokens=self.max_tokens,
                      device=self.device, schedule=self.schedule)
        self._models[mode] = (weights, model)
        return model

    def forget(self) -> None:
        """Drop the device caches, so the next call of every mode uploads its past rows afresh."""
        self._sequences.clear()

    def _cache_for(self, mode: str, model, past_keys: np.ndarray, past_values: np.ndarray, need: int):
        """The device cache for this call's sequence, holding the rows [0, past) of the host's;
        only rows it did not already hold are uploaded."""
        past = int(past_keys.shape[2])
        kbuf, vbuf = _owner(past_keys), _owner(past_values)
        seq = self._sequences.get(mode)
        fresh = seq is None or seq.keys_buffer is not kbuf or seq.values_buffer is not vbuf
        # a sequence's first call sizes the device cache for the whole host buffer (the reference's
        # preallocated one), so its later calls allocate nothing; a cache that must grow at least
        # doubles, so a growing sequence allocates O(log length) times
        want = max(need, _rows_of(kbuf, past_keys)) if fresh else need
        if seq is None or seq.cache.capacity < want:
            old = seq.cache.capacity if seq is not None else 0
            capacity = min(max(want, 2 * old if old < need else 0), MAX_CACHE_ROWS)
            if capacity < need:
                raise ValueError(f"{need} tokens exceed the device cache's limit of {MAX_CACHE_ROWS}")
            seq = _Sequence(model.new_cache(capacity))
            self._sequences[mode] = seq
            fresh = True                       # a new device cache holds nothing yet
        if fresh:
            seq.keys_buffer, seq.values_buffer, seq.held = kbuf, vbuf, 0
        seq.held = min(seq.held, past)         # a shorter view: the rows past it are not the caller's now
        if seq.held < past:
            _upload_rows(seq.cache.keys, past_keys, seq.held, past)
            _upload_rows(seq.cache.values, past_values, seq.held, past)
        seq.held = past
        seq.cache.length = past
        return seq

    def compiled(self, graph) -> "HIPCompiledGraph":
        """The graph bound once, on first use (the reference's CBackend.compiled, runtime.py:321-333)."""
        for held, bound in self._compiled:
            if held is graph:
                return bound
        bound = HIPCompiledGraph(graph, self.config, self.fuse, self.schedule, backend=self, device=self.device,
                                 lower=self.lower)
        self._compiled.append((graph, bound))
        return bound

    def __call__(self, graph, inputs: Mapping[str, np.ndarray], weights: Mapping[str, np.ndarray]) -> dict:
        return self.compiled(graph)(inputs, weights)

    def run(self, graph, mode: str, last_only: bool, inputs: Mapping[str, np.ndarray],
            weights: Mapping[str, np.ndarray]) -> dict:
        c = self.config
        ids = np.asarray(inputs["token_ids"], np.int64)
        past_keys = np.asarray(inputs["past_keys"], np.float32)
        past_values = np.asarray(inputs["past_values"], np.float32)
        layout = (c.num_hidden_layers, c.num_key_value_heads)
        if ids.ndim != 1 or ids.size == 0:
            raise ValueError(f"token_ids must be a non-empty 1-D array, got shape {ids.shape}")
        if (past_keys.shape[:2] != layout or past_keys.shape[3:] != (c.head_dim,)
                or past_values.shape != past_keys.shape):
            raise ValueError(f"past_keys / past_values of shapes {past_keys.shape} / {past_values.shape}; "
                             f"expected [{layout[0]}, {layout[1]}, past, {c.head_dim}]")
        m, past = int(ids.size), int(past_keys.shape[2])
        if m > self.max_tokens:
            raise ValueError(f"{m} tokens in one call; this backend was made with max_tokens={self.max_tokens}")
        model = self._model(mode, weights)
        seq = self._cache_for(mode, model, past_keys, past_values, past + m)
        logits = model.forward(ids, seq.cache, last_only=last_only)
        keys = _download_rows(seq.cache.keys, past, past + m)
        values = _download_rows(seq.cache.values, past, past + m)
        # the caller appends these at rows past .. past + m of the same buffer (models/qwen2.py:263-271)
        seq.held = past + m
        return {"logits": logits, "keys": keys, "values": values}


MAX_CACHE_ROWS = 16000          # the attention kernels' limit on positions, in every mode


class _Sequence:
    """A device cache and which host buffers its rows [0, held) mirror."""

    def __init__(self, cache) -> None:
        self.cache = cache
        self.keys_buffer = self.values_buffer = None
        self.held = 0


def _owner(view: np.ndarray) -> np.ndarray:
    """The array whose memory ``view`` starts, when it is a leading slice of it along the rows
    (the reference's ``_keys[:, :, :length]``); else the view itself. Identity of this array
    names the sequence."""
    root = view
    while isinstance(root.base, np.ndarray):
        root = root.base
    if (root is not view and root.ndim == 4 and root.shape[:2] == view.shape[:2] and root.shape[3] == view.shape[3]
            and root.strides == view.strides and root.ctypes.data == view.ctypes.data):
        return root
    return view


def _rows_of(buffer: np.ndarray, view: np.ndarray) -> int:
    """The host buffer's capacity in rows when ``view`` is its leading slice, else the view's rows."""
    return int(buffer.shape[2]) if buffer is not view else int(view.shape[2])


def _upload_rows(device, host: np.ndarray, start: int, stop: int) -> None:
    """Rows [start, stop) of every (layer, head) of ``host`` [L, kv, past, D] into the device cache
    [L, kv, capacity, D]: one strided copy when the host rows have a uniform pitch."""
    from nanocompile_amd import hip
    layers, heads, _, width = host.shape
    capacity = device.shape[2]
    row = width * 4
    if not (host.strides[3] == 4 and host.strides[2] == row and host.strides[0] == heads * host.strides[1]):
        host = np.ascontiguousarray(host[:, :, start:stop])
        start, stop = 0, host.shape[2]
        src = host.ctypes.data
    else:
        src = host.ctypes.data + start * row
    pitch = host.strides[1]
    hip.copy_rows(device.ptr + start * row, capacity * row, src, pitch, (stop - start) * row, layers * heads,
                  to_device=True)


def _download_rows(device, start: int, stop: int) -> np.ndarray:
    """Rows [start, stop) of every (layer, head) of the device cache, as a host [L, kv, n, D] array."""
    from nanocompile_amd import hip
    layers, heads, capacity, width = device.shape
    row = width * 4
    out = np.empty((layers, heads, stop - start, width), np.float32)
    if out.size:
        hip.copy_rows(out.ctypes.data, (stop - start) * row, device.ptr + start * row, capacity * row,
                      (stop - start) * row, layers * heads, to_device=False)
    return out


class HIPCompiledGraph:
    """A graph compiled for the GPU: the reference's ``CompiledGraph(graph, fuse, schedule)`` and its
    ``__call__(inputs, weights, bindings=None, profile=None) -> dict`` (runtime.py:167-301).

    Two paths, chosen once:

    * a Qwen2 forward graph of ``config`` (recognised by interface and int8 primitive) runs on the
      hand-written model library (models/qwen2.py), whose kernels compute the reference's bits for
      the projections and its operations in a stated order elsewhere; ``fuse`` does not change its
      result (the reference holds fused and unfused programs bitwise equal, test_codegen.py:40-52);
    * any other graph, or any ``program`` given, runs as generated HIP: the reference's compiled
      program (``fusion.fuse(passes.optimize(graph))``, or ``lower.lower(graph)`` with
      ``fuse=False``; its runtime.py:186) lowered by codegen_hip with GPU schedules, on one device
      arena (compiled.CompiledProgram). ``program`` may be the reference's Program or a recorded
      one (lir.program_from_json); ``lower(graph, fuse)`` may supply the compilation, else the
      reference's own passes are imported (the host framework a drop-in backend runs inside).

    ``schedule`` is ``"default"``, an ``autotune.Autotuner`` (on the model path it tunes the
    projections; on generated code each kernel over its GPU schedule space, the reference's
    ``CompiledGraph(graph, schedule=Autotuner())``), or for generated code a function
    ``(kernel, calls) -> (kernel, Launch)`` or an object with ``schedule_program(program)``. ``bindings``, when given, must agree with the
    inputs' symbols (``check_arguments``); ``profile`` accumulates seconds per primitive (generated
    code) or under "qwen2_forward" (the model path, one sequence of kernels).
    """

    def __init__(self, graph=None, config=None, fuse: bool = True, schedule="default",
                 backend: HIPBackend | None = None, max_tokens: int = 512, device: int = 0, *,
                 program=None, lower=None) -> None:
        self.graph, self.fuse, self.schedule = graph, fuse, schedule
        self.path = "codegen"
        if program is None and graph is not None and (backend is not None or config is not None):
            self.backend = backend or HIPBackend(config, max_tokens=max_tokens, device=device, schedule=schedule)
            try:
                self.mode = self.backend.mode(graph)
                self.last_only = self.backend.last_only(graph, self.mode)
                self.path = "model"
            except NotImplementedError:
                pass
        if self.path == "codegen":
            from nanocompile_amd.compiled import CompiledProgram
            if program is None:
                if graph is None:
                    raise ValueError("HIPCompiledGraph needs a graph or a compiled program")
                program = lower(graph, fuse) if lower is not None else _reference_compile(graph, fuse)
            self.program = CompiledProgram(program, schedule=schedule, device=device)

    def __call__(self, inputs: Mapping[str, np.ndarray], weights: Mapping[str, np.ndarray],
                 bindings: Mapping[str, int] | None = None, profile: dict[str, float] | None = None) -> dict:
        if self.path == "codegen":
            return self.program(inputs, weights, bindings, profile)
        if bindings:
            bound = {"seq": int(np.asarray(inputs["token_ids"]).shape[0]),
                     "past": int(np.asarray(inputs["past_keys"]).shape[2])}
            for name, value in bindings.items():
                if name not in bound or bound[name] != int(value):
                    raise ValueError(f"binding {name}={value} disagrees with the inputs ({bound})")
        started = time.perf_counter()
        out = self.backend.run(self.graph, self.mode, self.last_only, inputs, weights)
        if profile is not None:
            profile["qwen2_forward"] = profile.get("qwen2_forward", 0.0) + time.perf_counter() - started
        return out


def _reference_compile(graph, fuse: bool):
    """The reference's own compilation of ``graph`` (runtime.py:186): its passes, run where it is installed."""
    try:
        from nanocompile.fusion import fuse as fuse_graph
        from nanocompile.lower import lower
        from nanocompile.passes import optimize
    except ImportError as error:
        raise NotImplementedError(
            f"graph {getattr(graph, 'name', graph)!r} is not a Qwen2 forward this backend runs natively, and "
            f"the reference's compiler (nanocompile) is not importable to lower it; pass program= or lower=") \
            from error
    return fuse_graph(optimize(graph)) if fuse else lower(graph)
