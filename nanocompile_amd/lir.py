"""The reference's compiled programs as this package reads them: loop IR, calls, buffers, views.

A drop-in backend receives what the reference's compiler produces for a graph
(passes.optimize then fusion.fuse, lower.py:101-128): a Program of distinct
loop-IR kernels (loopir.py:329-345) and the ordered calls that run them on
views of buffers. The code generator (codegen_hip.py) and the runtime
(compiled.py) read those objects by their class names and fields, so they
take the reference's own objects unchanged; this module holds the same shapes
for programs that arrive as data (a JSON document, e.g. the recorded
programs the tests replay on a machine without the reference).

The node classes carry the reference's field names because those fields are
the interface; they only hold data, and nothing here rebuilds or folds IR.
Symbolic dimensions (shapes, strides, view offsets, traffic) are polynomials
in the graph's symbols (``seq``, ``past``): :class:`Poly` evaluates them.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

DTYPES = {"f32": np.dtype(np.float32), "i64": np.dtype(np.int64), "i32": np.dtype(np.int32),
          "i8": np.dtype(np.int8), "bool": np.dtype(np.bool_)}


# -- symbolic dimensions ------------------------------------------------------------------


@dataclass(frozen=True)
class Poly:
    """A polynomial with integer coefficients over named symbols: ``terms`` = ((coeff, (names...)), ...)."""

    terms: tuple[tuple[int, tuple[str, ...]], ...]

    def evaluate(self, bound) -> int:
        total = 0
        for coeff, names in self.terms:
            term = coeff
            for name in names:
                if name not in bound:
                    raise KeyError(f"no value bound for {name}")
                term *= int(bound[name])
            total += term
        return total

    @property
    def symbols(self) -> frozenset[str]:
        return frozenset(n for _, names in self.terms for n in names)

    def __str__(self) -> str:
        parts = ["*".join([str(c)] * (c != 1 or not m) + list(m)) for c, m in self.terms]
        return " + ".join(parts) or "0"


def evaluate(d, bound) -> int:
    """An int, a Poly, or anything with ``evaluate(bindings)`` (the reference's Expr), at ``bound``."""
    if isinstance(d, (int, np.integer)):
        return int(d)
    return int(d.evaluate(bound))


def shape_of(dims, bound) -> tuple[int, ...]:
    return tuple(evaluate(d, bound) for d in dims)


def as_symbol(d) -> str | None:
    """The symbol's name when ``d`` is exactly one symbol (``seq``), else None."""
    if isinstance(d, Poly):
        if len(d.terms) == 1 and d.terms[0][0] == 1 and len(d.terms[0][1]) == 1:
            return d.terms[0][1][0]
        return None
    return getattr(d, "as_symbol", None)


# -- loop IR (the reference's loopir.py node shapes) --------------------------------------


@dataclass(frozen=True)
class DType:
    name: str

    @property
    def numpy(self) -> np.dtype:
        return DTYPES[self.name]

    @property
    def is_float(self) -> bool:
        return self.name == "f32"

    @property
    def is_int(self) -> bool:
        return self.name in ("i64", "i32", "i8")


@dataclass(frozen=True)
class Const:
    value: object
    dtype: DType


@dataclass(frozen=True)
class Var:
    name: str
    dtype: DType = DType("i64")


@dataclass(frozen=True)
class Sym:
    index: int
    dtype: DType = DType("i64")


@dataclass(frozen=True)
class Load:
    param: int
    index: object
    dtype: DType


@dataclass(frozen=True)
class Binary:
    op: str
    a: object
    b: object
    dtype: DType


@dataclass(frozen=True)
class Unary:
    op: str
    a: object
    dtype: DType


@dataclass(frozen=True)
class Select:
    cond: object
    a: object
    b: object
    dtype: DType


@dataclass(frozen=True)
class Cast:
    a: object
    dtype: DType


@dataclass(frozen=True)
class Local:
    name: str
    index: object
    dtype: DType


@dataclass(frozen=True)
class Fma:
    a: object
    b: object
    c: object
    dtype: DType


@dataclass(frozen=True)
class Dp4:
    a: Load
    b: Load
    dtype: DType = DType("i32")


@dataclass(frozen=True)
class Loop:
    var: str
    extent: object
    body: tuple
    kind: str = "serial"


@dataclass(frozen=True)
class Store:
    param: int
    index: object
    value: object


@dataclass(frozen=True)
class Let:
    var: str
    value: object


@dataclass(frozen=True)
class Assign:
    var: str
    value: object


@dataclass(frozen=True)
class Fail:
    cond: object
    code: int


@dataclass(frozen=True)
class Array:
    name: str
    size: int
    init: Const


@dataclass(frozen=True)
class ArrayStore:
    name: str
    index: object
    value: object


@dataclass(frozen=True)
class Block:
    body: tuple


@dataclass(frozen=True)
class Param:
    dtype: DType
    writable: bool
    packed: int | None = None


@dataclass(frozen=True)
class Kernel:
    primitive: str
    params: tuple
    body: tuple
    bytes_read: object = field(default=0, compare=False)
    bytes_written: object = field(default=0, compare=False)


NODES = {c.__name__: c for c in (Const, Var, Sym, Load, Binary, Unary, Select, Cast, Local, Fma, Dp4, Loop,
                                 Store, Let, Assign, Fail, Array, ArrayStore, Block)}


# -- programs ----------------------------------------------------------------------------------


class Buffer:
    """Storage for one value: ``kind`` is input, weight, const, temp or output (lower.py's Buffer)."""

    __slots__ = ("kind", "name", "dtype", "shape", "value")

    def __init__(self, kind: str, dtype: DType, shape: tuple, name: str | None = None, value=None) -> None:
        self.kind, self.dtype, self.shape, self.name, self.value = kind, dtype, shape, name, value

    def __repr__(self) -> str:
        return f"<Buffer {self.kind} {self.name or ''} {self.dtype.name}{list(map(str, self.shape))}>"


@dataclass(frozen=True)
class View:
    buffer: Buffer
    shape: tuple
    strides: tuple
    offset: object

    @property
    def dtype(self) -> DType:
        return self.buffer.dtype


@dataclass(frozen=True)
class Call:
    kernel: int
    output: Buffer
    operands: tuple
    primitive: str
    node: int
    op: str = ""
    gather: dict | None = None      # rows and the ids input, for a gather's error message


@dataclass
class Program:
    """Kernels and calls (lower.py:101-128), with the graph's interface a runtime needs."""

    name: str
    symbols: tuple[str, ...]
    inputs: list[tuple[str, DType, tuple]]             # (name, dtype, shape), in the graph's order
    weights: dict[str, tuple[DType, tuple]]
    kernels: list[Kernel]
    calls: list[Call]
    buffers: list[Buffer]
    outputs: dict[str, Buffer]
    bytes_moved: object = 0

    def last_uses(self) -> dict[Buffer, int]:
        """Each temp buffer's last reading call (a temp nobody reads dies at the call that writes it)."""
        last: dict[Buffer, int] = {}
        for index, call in enumerate(self.calls):
            if call.output.kind == "temp":
                last.setdefault(call.output, index)
            for view in call.operands:
                if view.buffer.kind == "temp":
                    last[view.buffer] = index
        return last


def adapt(program) -> Program:
    """This module's Program for the reference's own (lower.py:101-128, a graph attached): the graph's
    interface and each gather's operands read off its nodes; kernels, buffers and views kept as they are."""
    if isinstance(program, Program):
        return program
    g = program.graph
    inputs = [(n.attrs["name"], n.dtype, tuple(n.shape)) for n in g.inputs]
    weights = {name: (n.dtype, tuple(n.shape)) for name, n in g.weights.items()}
    calls = []
    for c in program.calls:
        node = g.nodes[c.node]
        gather = None
        if node.op == "gather":
            table, ids = node.inputs
            gather = {"rows": table.shape[0], "ids_input": ids.attrs["name"] if ids.op == "input" else None}
        calls.append(Call(c.kernel, c.output, tuple(c.operands), c.primitive, c.node, node.op, gather))
    return Program(g.name, tuple(program.symbols), inputs, weights, list(program.kernels), calls,
                   list(program.buffers), dict(program.outputs), program.bytes_moved)


# -- reading the JSON form -------------------------------------------------------------------


def _dim(d):
    if isinstance(d, dict):
        return Poly(tuple((int(c), tuple(m)) for c, m in d["poly"]))
    return int(d)


def _node(obj):
    if isinstance(obj, list):
        return tuple(_node(x) for x in obj)
    if not isinstance(obj, dict):
        return obj
    kind = obj["_"]
    if kind == "Const":
        dtype = DType(obj["dtype"])
        v = obj["value"]
        value = float.fromhex(v["f"]) if isinstance(v, dict) else int(v)
        return Const(value, dtype)
    cls = NODES[kind]
    args = {}
    for name, value in obj.items():
        if name == "_":
            continue
        if name == "dtype":
            args[name] = DType(value)
        else:
            args[name] = _node(value)
    return cls(**args)


def kernel_from_json(k: dict) -> Kernel:
    params = tuple(Param(DType(p["dtype"]), bool(p["writable"]), p["packed"]) for p in k["params"])
    return Kernel(k["primitive"], params, tuple(_node(s) for s in k["body"]), _dim(k["bytes_read"]),
                  _dim(k["bytes_written"]))


def program_from_json(doc: dict, arrays=None) -> Program:
    """A Program from its JSON form; ``arrays`` maps the names of constant buffers' values to arrays."""
    buffers = []
    for b in doc["buffers"]:
        value = None
        if b["kind"] == "const":
            value = np.asarray(arrays[b["value"]])
        buffers.append(Buffer(b["kind"], DType(b["dtype"]), tuple(_dim(d) for d in b["shape"]), b["name"], value))
    calls = []
    for c in doc["calls"]:
        operands = tuple(View(buffers[v["buffer"]], tuple(_dim(d) for d in v["shape"]),
                              tuple(_dim(d) for d in v["strides"]), _dim(v["offset"])) for v in c["operands"])
        gather = None
        if c.get("gather"):
            gather = {"rows": _dim(c["gather"]["rows"]), "ids_input": c["gather"]["ids_input"]}
        calls.append(Call(c["kernel"], buffers[c["output"]], operands, c["primitive"], c["node"], c.get("op", ""),
                          gather))
    return Program(
        name=doc["graph"], symbols=tuple(doc["symbols"]),
        inputs=[(i["name"], DType(i["dtype"]), tuple(_dim(d) for d in i["shape"])) for i in doc["inputs"]],
        weights={n: (DType(w["dtype"]), tuple(_dim(d) for d in w["shape"])) for n, w in doc["weights"].items()},
        kernels=[kernel_from_json(k) for k in doc["kernels"]], calls=calls, buffers=buffers,
        outputs={n: buffers[i] for n, i in doc["outputs"].items()}, bytes_moved=_dim(doc.get("bytes_moved", 0)))


def load_programs(path: str | Path) -> dict:
    """The JSON document of recorded programs (``.json`` or gzip-compressed ``.json.gz``)."""
    path = Path(path)
    if path.suffix == ".gz":
        import gzip
        with gzip.open(path, "rt", encoding="utf-8") as f:
            return json.load(f)
    return json.loads(path.read_text(encoding="utf-8"))
