"""Writes programs.json.gz and programs.npz: the reference's compiled programs, as data, with their outputs.

Run in the build container only, where /root/reference is mounted:

    python tests/golden/make_programs.py

The reference compiles a graph (ir.Graph) by optimizing and fusing it into a
Program (lower.py:101-128): distinct loop-IR kernels (loopir.py:329-345), the
ordered calls that run them on views of buffers, and the graph's interface.
That Program is what a GPU code generator consumes in place of the reference's
C emitter (runtime.py:182-200), so this script records it for a set of graphs:

* a zoo of small graphs covering every primitive the fused programs use
  (unary and binary arithmetic in each dtype, select and cast, reductions
  with NaN, rms_norm, softmax with the causal mask, RoPE, a linear layer,
  gather with its bounds check, concat with symbolic lengths, the int8 and
  int8-vnni projections of quantize.py with a SwiGLU block, rms_norm then a
  per-row int8 scale at width 896, config 2), each with seeded
  inputs at several symbol bindings and the outputs of the reference's
  compiled C (CompiledGraph, runtime.py:167-301) on them;
* the seeded tiny Qwen2 (the golden G5 model) in float32, int8 and
  int8-vnni, both forward graphs, whose tokens and logits G5 already holds;
* config 5's model, Qwen2.5-0.5B-shaped (24 layers, vocabulary 151,936) with
  BASELINE's seeded N(0, 0.02) weights, in int8: its last-position forward
  program, a seeded 16-token prompt, the reference's four greedy tokens
  from it, and the reference's logits of the prompt and of the first decode
  step at every 97th vocabulary entry and at the argmax (``--add config5``
  records only this entry, keeping the rest of the fixture as it is).

Each program is recorded fused and unscheduled (what the GPU schedules
start from); some also unfused (``lower``) and with the reference's CPU
schedules applied (vector and parallel loops, privatized accumulators), so
the code generator is exercised on every statement kind. The fixture is data
(loop trees, shapes as polynomials, numbers); no source of the reference is
copied.
"""

from __future__ import annotations

import gzip
import json
import os
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
REFERENCE = Path(os.environ.get("NANOCOMPILE_REFERENCE", "/root/reference"))
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(REFERENCE))
os.environ.setdefault("NANOCOMPILE_CACHE", tempfile.mkdtemp(prefix="nanocompile-cache-"))

from nanocompile import dtypes, nn, quantize  # noqa: E402  (the reference)
from nanocompile import loopir as L  # noqa: E402
from nanocompile.frontend import GraphBuilder, concat, gather, where  # noqa: E402
from nanocompile.fusion import fuse  # noqa: E402
from nanocompile.lower import lower  # noqa: E402
from nanocompile.models.qwen2 import Qwen2, Qwen2Config  # noqa: E402
from nanocompile.passes import optimize  # noqa: E402
from nanocompile.runtime import CompiledGraph  # noqa: E402
from nanocompile.schedule import schedule_program  # noqa: E402
from nanocompile import schedules  # noqa: E402
from nanocompile.symbolic import Expr  # noqa: E402

from nanocompile_amd.models import config as ours  # noqa: E402  (the seeded weight generator)

ARRAYS: dict[str, np.ndarray] = {}


# -- encoding ---------------------------------------------------------------------------------


def dim(d) -> object:
    """An int, or a polynomial as [[coefficient, [symbol, ...]], ...]."""
    if isinstance(d, (int, np.integer)):
        return int(d)
    assert isinstance(d, Expr), d
    return {"poly": [[int(c), list(m)] for m, c in d.terms()]}


def scalar_value(value, dtype) -> object:
    if dtype.is_float:
        return {"f": float(value).hex()}
    return int(value)


def node(x) -> object:
    """A loop-IR node (loopir.py) as JSON: its class name and fields."""
    if isinstance(x, L.Const):
        return {"_": "Const", "value": scalar_value(x.value, x.dtype), "dtype": x.dtype.name}
    if isinstance(x, (L.Var, L.Sym, L.Load, L.Binary, L.Unary, L.Select, L.Cast, L.Local, L.Fma, L.Dp4,
                      L.Loop, L.Store, L.Let, L.Assign, L.Fail, L.Array, L.ArrayStore, L.Block)):
        out = {"_": type(x).__name__}
        for name in x.__dataclass_fields__:
            out[name] = encode(getattr(x, name))
        return out
    raise TypeError(f"not a loop-IR node: {x!r}")


def encode(v):
    if isinstance(v, dtypes.DType):
        return v.name
    if isinstance(v, tuple):
        return [encode(x) for x in v]
    if isinstance(v, (str, bool)) or v is None:
        return v
    if isinstance(v, (int, np.integer)):
        return int(v)
    return node(v)


def kernel(k: L.Kernel) -> dict:
    return {"primitive": k.primitive,
            "params": [{"dtype": p.dtype.name, "writable": p.writable, "packed": p.packed} for p in k.params],
            "body": [node(s) for s in k.body],
            "bytes_read": dim(k.bytes_read), "bytes_written": dim(k.bytes_written)}


def program(p, key: str) -> dict:
    buffers = {id(b): i for i, b in enumerate(p.buffers)}
    out_buffers = []
    for i, b in enumerate(p.buffers):
        entry = {"kind": b.kind, "name": b.name, "dtype": b.dtype.name, "shape": [dim(d) for d in b.shape]}
        if b.kind == "const":
            ARRAYS[f"{key}/const{i}"] = np.asarray(b.value)
            entry["value"] = f"{key}/const{i}"
        out_buffers.append(entry)
    calls = []
    for c in p.calls:
        n = p.graph.nodes[c.node]
        call = {"kernel": c.kernel, "output": buffers[id(c.output)], "primitive": c.primitive, "node": c.node,
                "op": n.op,
                "operands": [{"buffer": buffers[id(v.buffer)], "shape": [dim(d) for d in v.shape],
                              "strides": [dim(d) for d in v.strides], "offset": dim(v.offset)}
                             for v in c.operands]}
        if n.op == "gather":
            table, ids = n.inputs
            call["gather"] = {"rows": dim(table.shape[0]),
                              "ids_input": ids.attrs["name"] if ids.op == "input" else None}
        calls.append(call)
    g = p.graph
    return {
        "graph": g.name,
        "symbols": list(p.symbols),
        "inputs": [{"name": n.attrs["name"], "dtype": n.dtype.name, "shape": [dim(d) for d in n.shape]}
                   for n in g.inputs],
        "weights": {name: {"dtype": n.dtype.name, "shape": [dim(d) for d in n.shape]}
                    for name, n in g.weights.items()},
        "kernels": [kernel(k) for k in p.kernels],
        "calls": calls,
        "buffers": out_buffers,
        "outputs": {name: buffers[id(b)] for name, b in p.outputs.items()},
        "bytes_moved": dim(p.bytes_moved),
    }


# -- the zoo ------------------------------------------------------------------------------------


def rand(rng, shape, dtype=np.float32):
    dtype = np.dtype(dtype)
    if dtype.kind == "f":
        return rng.standard_normal(shape).astype(dtype)
    if dtype.kind == "b":
        return rng.random(shape) > 0.5
    return rng.integers(-100, 100, size=shape).astype(dtype)


def zoo():
    """(name, graph, weights, [input dicts]) for each small graph."""
    rng = np.random.default_rng(2024)
    out = []

    b = GraphBuilder("unary")
    x = b.input("x", dtypes.f32, (b.symbol("seq"), 5))
    mag = where(0.0 <= x, x, -x)
    g = b.build({"neg": -x, "sqrt": mag.sqrt(), "reciprocal": x.reciprocal(), "round": (x * 4.0).round(),
                 "exp": x.exp(), "sin": (x * 3.0).sin(), "cos": (x * 3.0).cos()})
    out.append(("unary", g, {}, [{"x": rand(rng, (s, 5)) * 2} for s in (1, 3, 7)]))

    for dt in (dtypes.f32, dtypes.i32, dtypes.i8, dtypes.i64):
        b = GraphBuilder(f"binary_{dt.name}")
        s = b.symbol("seq")
        x, y = b.input("x", dt, (s, 6)), b.input("y", dt, (s, 6))
        outs = {"add": x + y, "sub": x - y, "mul": x * y, "le": x <= y}
        if dt.is_float:
            outs["div"] = x / y
        out.append((f"binary_{dt.name}", b.build(outs), {},
                    [{"x": rand(rng, (n, 6), dt.numpy), "y": rand(rng, (n, 6), dt.numpy)} for n in (1, 3, 7)]))

    b = GraphBuilder("where_cast")
    s = b.symbol("seq")
    c, x, n = b.input("c", dtypes.bool_, (s, 4)), b.input("x", dtypes.f32, (s, 4)), b.input("n", dtypes.i64, (s,))
    g = b.build({"w": where(c, x, -x), "f": n.cast(dtypes.f32), "q": n.cast(dtypes.i8), "back": x.cast(dtypes.i32),
                 "flag": n.cast(dtypes.bool_), "from_bool": c.cast(dtypes.f32)})
    out.append(("where_cast", g, {}, [{"c": rand(rng, (5, 4), np.bool_), "x": rand(rng, (5, 4)) * 50,
                                       "n": np.array([0, 1, 300, -3, 2**24 + 1], np.int64)}]))

    b = GraphBuilder("reductions")
    x = b.input("x", dtypes.f32, (b.symbol("seq"), 33))
    g = b.build({"s0": x.sum(0), "m0": x.max(0), "s1": x.sum(1), "m1": x.max(-1)})
    cases = [{"x": rand(rng, (s, 33))} for s in (1, 3, 7)]
    nan = rand(rng, (3, 33))
    nan[1, 5] = np.nan
    nan[2] = -np.inf
    cases.append({"x": nan})
    out.append(("reductions", g, {}, cases))

    b = GraphBuilder("rms_norm")
    x = b.input("x", dtypes.f32, (b.symbol("seq"), 96))
    g = b.build({"y": nn.rms_norm(x, b.weight("w", (96,)), 1e-6)})
    out.append(("rms_norm", g, {"w": (1 + 0.1 * rand(rng, (96,))).astype(np.float32)},
                [{"x": rand(rng, (s, 96))} for s in (1, 3, 7)]))

    b = GraphBuilder("softmax_mask")
    seq, past = b.symbol("seq"), b.symbol("past")
    sc = b.input("s", dtypes.f32, (2, seq, past + seq))
    anchor = b.input("anchor", dtypes.f32, (past,))           # binds past
    g = b.build({"p": nn.softmax(sc + nn.causal_mask(b, seq, past), axis=-1), "n": anchor * 1.0})
    out.append(("softmax_mask", g, {}, [{"s": rand(rng, (2, q, p + q)) * 3, "anchor": rand(rng, (p,))}
                                        for q, p in ((1, 0), (1, 12), (5, 3))]))

    b = GraphBuilder("rope")
    seq, past = b.symbol("seq"), b.symbol("past")
    x = b.input("x", dtypes.f32, (2, seq, 8))
    anchor = b.input("anchor", dtypes.f32, (past,))
    positions = b.iota((seq,), axis=0) + b.dim(past)
    cos, sin = nn.rope_tables(positions, 8, 1e6)
    g = b.build({"y": nn.apply_rope(x, cos, sin), "n": anchor * 1.0})
    out.append(("rope", g, {}, [{"x": rand(rng, (2, q, 8)), "anchor": rand(rng, (p,))}
                                for q, p in ((1, 0), (3, 5), (2, 700))]))

    b = GraphBuilder("linear")
    x = b.input("x", dtypes.f32, (b.symbol("seq"), 40))
    g = b.build({"y": nn.linear(x, b.weight("w", (24, 40)), b.weight("bias", (24,)))})
    out.append(("linear", g, {"w": rand(rng, (24, 40)) * 0.2, "bias": rand(rng, (24,))},
                [{"x": rand(rng, (s, 40))} for s in (1, 3, 7)]))

    b = GraphBuilder("gather")
    ids = b.input("ids", dtypes.i64, (b.symbol("seq"),))
    table = b.weight("table", (50, 8))
    g = b.build({"rows": gather(table, ids) * 2.0})
    out.append(("gather", g, {"table": rand(rng, (50, 8))},
                [{"ids": np.array(v, np.int64)} for v in ([3], [0, 49, 7], [5, 50, 2], [-1])]))

    b = GraphBuilder("concat_kv")
    seq, past = b.symbol("seq"), b.symbol("past")
    old = b.input("old", dtypes.f32, (2, past, 4))
    new = b.input("new", dtypes.f32, (2, seq, 4))
    both = concat([old, new], axis=1)
    g = b.build({"all": both, "total": both.sum(1)})
    out.append(("concat_kv", g, {}, [{"old": rand(rng, (2, p, 4)), "new": rand(rng, (2, q, 4))}
                                     for q, p in ((1, 0), (1, 6), (4, 3))]))

    # int8-vnni quantizes every activation in blocks of 32: both widths must be multiples of 32
    for mode, shapes in (("int8", ((64, 40), (96, 24), (160, 40))), ("int8-vnni", ((64, 32), (96, 64), (128, 32)))):
        for k, n_out in shapes:
            b = GraphBuilder(f"mlp_{mode}_{k}")
            x = b.input("x", dtypes.f32, (b.symbol("seq"), k))
            gate = nn.linear(x, b.weight("gate", (n_out, k)))
            up = nn.linear(x, b.weight("up", (n_out, k)))
            h = nn.silu(gate) * up
            y = nn.linear(h, b.weight("down", (k, n_out)), b.weight("bias", (k,)))
            graph = b.build({"y": y + x})
            acts = "f32" if mode == "int8" else "int8"
            graph = quantize.quantize(graph, acts)
            w = {"gate": rand(rng, (n_out, k)) * 0.2, "up": rand(rng, (n_out, k)) * 0.2,
                 "down": rand(rng, (k, n_out)) * 0.2, "bias": rand(rng, (k,))}
            weights = quantize.quantized_weights(graph, w)
            out.append((f"mlp_{mode}_{k}", graph, weights, [{"x": rand(rng, (s, k))} for s in (1, 3, 7)]))

    # config 2 written in the reference's graph ops: rms_norm, then one int8 scale per row
    # (quantize_activations' steps, quantize.py:102-124, with one block spanning the 896-wide
    # row, which its power-of-two block cannot express); its unfused lowering is the
    # multi-kernel form the fused kernel is compared with
    b = GraphBuilder("rms_norm_quant")
    x = b.input("x", dtypes.f32, (b.symbol("seq"), 896))
    y = nn.rms_norm(x, b.weight("w", (896,)), 1e-6)
    magnitude = where(0.0 <= y, y, -y).max(-1)
    scale = where(magnitude <= 0.0, 1.0, magnitude / 127.0)
    rounded = (y / scale).round()
    clamped = where(rounded <= 127.0, rounded, 127.0)
    clamped = where(-127.0 <= clamped, clamped, -127.0)
    g = b.build({"normed": y, "xq": clamped.cast(dtypes.i8), "xs": scale * 1.0})
    cases = []
    for s in (1, 3, 7):
        v = rand(rng, (s, 896))
        v[rng.random(v.shape) < 0.01] *= 20
        cases.append({"x": v})
    out.append(("rms_norm_quant", g, {"w": (1 + 0.1 * rand(rng, (896,))).astype(np.float32)}, cases))
    return out


def record_zoo(fixture: dict) -> None:
    for name, graph, weights, cases in zoo():
        fused = fuse(optimize(graph))
        entry = {"program": program(fused, f"{name}/fused"), "unfused": program(lower(graph), f"{name}/unfused"),
                 "scheduled": program(schedule_program(fused, schedules.default), f"{name}/scheduled"),
                 "cases": []}
        for w, value in weights.items():
            ARRAYS[f"{name}/weight/{w}"] = np.asarray(value)
        compiled = CompiledGraph(graph, schedule=None)
        for i, inputs in enumerate(cases):
            case = {"inputs": {}, "outputs": {}}
            for k, v in inputs.items():
                ARRAYS[f"{name}/case{i}/in/{k}"] = v
                case["inputs"][k] = f"{name}/case{i}/in/{k}"
            try:
                result = compiled(inputs, weights)
            except Exception as error:                 # the reference's KernelError (gather out of range)
                case["error"] = f"{type(error).__name__}: {error}"
            else:
                for k, v in result.items():
                    ARRAYS[f"{name}/case{i}/out/{k}"] = v
                    case["outputs"][k] = f"{name}/case{i}/out/{k}"
            entry["cases"].append(case)
        entry["weights"] = {w: f"{name}/weight/{w}" for w in weights}
        fixture["zoo"][name] = entry
        print(f"{name}: {len(fused.kernels)} kernels, {len(fused.calls)} calls, {len(cases)} cases", flush=True)


def record_qwen2(fixture: dict) -> None:
    c = ours.TINY
    config = Qwen2Config(c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
                         c.num_attention_heads, c.num_key_value_heads, c.rms_norm_eps, c.rope_theta,
                         c.tie_word_embeddings)
    weights = ours.random_weights(c, seed=5, std=ours.TINY_STD)
    for mode in (None, "int8", "int8-vnni"):
        tag = {None: "f32", "int8": "int8", "int8-vnni": "vnni"}[mode]
        model = Qwen2(config, weights, quantization=mode)
        entry = {}
        for which, graph in (("full", model.graph), ("last", model.graph_last)):
            fused = fuse(optimize(graph))
            entry[which] = program(fused, f"qwen2_{tag}/{which}")
            print(f"qwen2 {tag} {which}: {len(fused.kernels)} kernels, {len(fused.calls)} calls", flush=True)
        if mode == "int8":
            entry["last_scheduled"] = program(schedule_program(fuse(optimize(model.graph_last)), schedules.default),
                                              f"qwen2_{tag}/last_scheduled")
        if mode is None:
            entry["last_unfused"] = program(lower(model.graph_last), f"qwen2_{tag}/last_unfused")
        entry["weight_names"] = sorted(model.weights)
        fixture["qwen2"][tag] = entry


CONFIG5_SEED, CONFIG5_PROMPT_SEED, CONFIG5_PROMPT, CONFIG5_NEW = 7, 11, 16, 4
CONFIG5_STRIDE = 97                     # logits recorded at every 97th vocabulary entry


def record_config5(fixture: dict) -> None:
    from nanocompile.models.qwen2 import greedy
    c = ours.QWEN25_05B
    config = Qwen2Config(c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
                         c.num_attention_heads, c.num_key_value_heads, c.rms_norm_eps, c.rope_theta,
                         c.tie_word_embeddings)
    model = Qwen2(config, ours.random_weights(c, seed=CONFIG5_SEED), quantization="int8")
    prompt = [int(t) for t in np.random.default_rng(CONFIG5_PROMPT_SEED).integers(0, c.vocab_size, CONFIG5_PROMPT)]
    fused = fuse(optimize(model.graph_last))
    entry = {"last": program(fused, "config5/last"), "weight_names": sorted(model.weights),
             "seed": CONFIG5_SEED, "prompt": prompt, "stride": CONFIG5_STRIDE}
    cache = model.new_cache(CONFIG5_PROMPT + CONFIG5_NEW)
    first = model.forward(prompt, cache=cache, last_only=True)[0]
    step = model.forward([int(np.argmax(first))], cache=cache, last_only=True)[0]
    for name, logits in (("prompt", first), ("step", step)):
        ARRAYS[f"config5/logits_{name}"] = np.ascontiguousarray(logits[::CONFIG5_STRIDE])
        entry[f"argmax_{name}"] = int(np.argmax(logits))
        entry[f"max_{name}"] = float(np.max(logits)).hex()
    entry["tokens"] = greedy(model, prompt, CONFIG5_NEW)
    print(f"config5: {len(fused.kernels)} kernels, {len(fused.calls)} calls, tokens {entry['tokens']}", flush=True)
    fixture["config5"] = entry


def main() -> None:
    if sys.argv[1:] == ["--add", "config5"]:
        with gzip.open(HERE / "programs.json.gz", "rt", encoding="utf-8") as f:
            fixture = json.load(f)
        record_config5(fixture)
    else:
        fixture = {"zoo": {}, "qwen2": {}}
        record_zoo(fixture)
        record_qwen2(fixture)
        record_config5(fixture)
    with gzip.open(HERE / "programs.json.gz", "wt", encoding="utf-8", compresslevel=9) as f:
        json.dump(fixture, f, sort_keys=True)
    # Arrays already in the fixture are kept: a re-run adds new entries without moving the
    # old ones. (On one host the reference's C gave 0 for sqrt(where(0 <= x, x, -x)) at four
    # negative x of unary case 2, where the recorded run gave sqrt(|x|); the recorded values
    # are the mathematically right ones and stay.)
    if (HERE / "programs.npz").exists():
        with np.load(HERE / "programs.npz", allow_pickle=False) as old:
            for key in old.files:
                if key in ARRAYS and not np.array_equal(old[key], ARRAYS[key], equal_nan=True):
                    print(f"{key}: this run's reference output differs from the recorded one; keeping the recorded")
                ARRAYS[key] = old[key]
    np.savez_compressed(HERE / "programs.npz", **ARRAYS)
    print(f"wrote programs.json.gz ({(HERE / 'programs.json.gz').stat().st_size // 1024} KiB) and programs.npz "
          f"({(HERE / 'programs.npz').stat().st_size // 1024} KiB, {len(ARRAYS)} arrays)")


if __name__ == "__main__":
    main()
