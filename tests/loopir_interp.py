"""A bounds-checked CPU interpreter of loop IR, for checking generated kernels before they reach a GPU.

TEST INFRASTRUCTURE. Each kernel (the reference's loop IR, as scheduled for
the GPU: packed, simplified) is rendered to a Python function with C's
scalar meaning (the meaning the reference's C and this package's HIP give
it): float32 arithmetic rounded per operation, C's integer promotion and
wrapping, truncating division, ``fmaf`` rounded once (the product exact in
float64, the sum rounded to float32 from it), ``roundf`` half away from
zero, and exp/sin/cos from the host build of csrc/nc_math.h (the GPU's own
functions). Every load, store and local-array access is range-checked
against the buffer the runtime would hand the kernel: an index outside it
raises instead of reading or writing out of bounds, which on a GPU is a
memory fault. Programs run call by call on NumPy buffers.
"""

from __future__ import annotations

import numpy as np

from nanocompile_amd import gpu_schedule, lir
from nanocompile_amd.compiled import pack_rows

F = np.float32


class OutOfBounds(IndexError):
    """A kernel indexed outside its operand."""


def _kind(x) -> str:
    return type(x).__name__


def _wrap(v: int, bits: int) -> int:
    m = 1 << bits
    return ((v + (m >> 1)) % m) - (m >> 1)


def _cdiv(a: int, b: int) -> int:
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


def _cmod(a: int, b: int) -> int:
    return a - _cdiv(a, b) * b


def _math(kind: str, x):
    from oracle import host
    return host.math("nc_" + kind, np.array([x], F))[0]


def _round(x):
    if not np.isfinite(x) or abs(float(x)) >= 2.0**23:
        return F(x)
    v = float(x)
    return F(np.copysign(np.floor(abs(v) + 0.5), v))


def _fma(a, b, c):
    return F(np.float64(a) * np.float64(b) + np.float64(c))


WIDTH = {"i64": 64, "i32": 32, "i8": 8}


class _Py:
    """Python source for one kernel."""

    def __init__(self, out_type: str) -> None:
        self.consts: list = []
        self.out_type = out_type

    def const(self, c) -> str:
        if c.dtype.name == "f32":
            self.consts.append(F(c.value))
            return f"K[{len(self.consts) - 1}]"
        return str(int(c.value))

    def x(self, e) -> tuple[str, str]:
        """(source, dtype name) of a scalar."""
        k = _kind(e)
        if k == "Const":
            return self.const(e), e.dtype.name
        if k == "Var":
            return e.name, e.dtype.name
        if k == "Sym":
            return f"S[{e.index}]", "i64"
        if k == "Load":
            idx, _ = self.x(e.index)
            return f"LD(X[{e.param}], {idx})", e.dtype.name
        if k == "Local":
            idx, _ = self.x(e.index)
            return f"LL({e.name}, {idx})", e.dtype.name
        if k == "Cast":
            a, t = self.x(e.a)
            to = e.dtype.name
            if to == "f32":
                return f"F({a})", to
            if to == "bool":
                return (f"(int({a}) & 255)" if t != "f32" else f"(CI({a}) & 255)"), to
            if t == "f32":
                return f"W(CI({a}), {WIDTH[to]})", to
            return f"W(int({a}), {WIDTH[to]})", to
        if k == "Select":
            c, _ = self.x(e.cond)
            a, _ = self.x(e.a)
            b, _ = self.x(e.b)
            return f"({a} if {c} else {b})", e.dtype.name
        if k == "Fma":
            return f"FMA({self.x(e.a)[0]}, {self.x(e.b)[0]}, {self.x(e.c)[0]})", "f32"
        if k == "Dp4":
            a, b = e.a, e.b
            return f"DP4(X[{a.param}], {self.x(a.index)[0]}, X[{b.param}], {self.x(b.index)[0]})", "i32"
        if k == "Unary":
            a, t = self.x(e.a)
            if e.op == "neg":
                return (f"(-{a})" if t == "f32" else f"W(-{a}, {max(32, WIDTH.get(t, 32))})"), t
            if e.op == "reciprocal":
                return f"(F(1.0) / {a})", t
            if e.op == "sqrt":
                return f"F(np.sqrt({a}))", t
            if e.op == "round":
                return f"RND({a})", t
            return f"M('{e.op}', {a})", t
        if k == "Binary":
            a, t = self.x(e.a)
            b, _ = self.x(e.b)
            op = e.op
            if op in ("le", "lt", "ne"):
                sym = {"le": "<=", "lt": "<", "ne": "!="}[op]
                return f"(1 if {a} {sym} {b} else 0)", "bool"
            if op == "or":
                return f"(1 if ({a} or {b}) else 0)", "bool"
            if t == "f32":
                sym = {"add": "+", "sub": "-", "mul": "*", "div": "/"}[op]
                return f"({a} {sym} {b})", t
            bits = 64 if t == "i64" else 32
            if op == "idiv":
                return f"W(CDIV({a}, {b}), {bits})", t
            if op == "mod":
                return f"W(CMOD({a}, {b}), {bits})", t
            sym = {"add": "+", "sub": "-", "mul": "*"}[op]
            return f"W({a} {sym} {b}, {bits})", t
        raise TypeError(f"cannot interpret {e!r}")

    def conv(self, src: str, t: str) -> str:
        """A value converted to a variable or element of type ``t`` (C's assignment)."""
        if t == "f32":
            return f"F({src})"
        if t == "bool":
            return f"(int({src}) & 255)"
        return f"W(int({src}), {WIDTH[t]})"

    def stmts(self, stmts, depth: int, types: dict) -> list[str]:
        pad = "    " * depth
        out = []
        for s in stmts:
            k = _kind(s)
            if k == "Loop":
                ext, _ = self.x(s.extent)
                out.append(f"{pad}for {s.var} in range({ext}):")
                body = self.stmts(s.body, depth + 1, types)
                out += body or [f"{pad}    pass"]
            elif k == "Block":
                out += self.stmts(s.body, depth, types)
            elif k == "Store":
                idx, _ = self.x(s.index)
                val, t = self.x(s.value)
                out.append(f"{pad}ST(X[0], {idx}, {self.conv(val, self.out_type)})")
            elif k == "Let":
                val, t = self.x(s.value)
                types[s.var] = t
                out.append(f"{pad}{s.var} = {self.conv(val, t)}")
            elif k == "Assign":
                val, t = self.x(s.value)
                out.append(f"{pad}{s.var} = {self.conv(val, types.get(s.var, t))}")
            elif k == "Fail":
                c, _ = self.x(s.cond)
                out.append(f"{pad}if {c}:")
                out.append(f"{pad}    return {s.code}")
            elif k == "Array":
                size = s.size if isinstance(s.size, int) else f"int({self.x(s.size)[0]})"
                out.append(f"{pad}{s.name} = [{self.const(s.init)}] * {size}")
            elif k == "ArrayStore":
                idx, _ = self.x(s.index)
                val, t = self.x(s.value)
                out.append(f"{pad}SL({s.name}, {idx}, {self.conv(val, t)})")
            else:
                raise TypeError(f"cannot interpret {s!r}")
        return out


def _ld(a, i):
    if not 0 <= i < a.size:
        raise OutOfBounds(f"load at {i} of an operand of {a.size} elements")
    v = a[i]
    return v if a.dtype == np.float32 else int(v)


def _st(a, i, v):
    if not 0 <= i < a.size:
        raise OutOfBounds(f"store at {i} of an output of {a.size} elements")
    a[i] = v


def _ll(arr, i):
    if not 0 <= i < len(arr):
        raise OutOfBounds(f"local read at {i} of {len(arr)}")
    return arr[i]


def _sl(arr, i, v):
    if not 0 <= i < len(arr):
        raise OutOfBounds(f"local write at {i} of {len(arr)}")
    arr[i] = v


def _ci(v):
    if not np.isfinite(v):
        raise OverflowError("a float that is not finite cast to an integer")
    return int(v)


def _dp4(a, i, b, j):
    total = 0
    for q in range(4):
        total += (_ld(a, i + q) + 128) * _ld(b, j + q)
    return total


ENV = {"F": F, "np": np, "LD": _ld, "ST": _st, "LL": _ll, "SL": _sl, "W": _wrap, "CDIV": _cdiv, "CMOD": _cmod,
       "CI": _ci, "FMA": _fma, "DP4": _dp4, "RND": _round, "M": _math}


def compile_kernel(kernel):
    """A Python function ``fn(X, S) -> 0 or a Fail code`` for one kernel."""
    py = _Py(kernel.params[0].dtype.name)
    body = py.stmts(kernel.body, 1, {})
    source = "def kernel(X, S, K):\n" + "\n".join(body or ["    pass"]) + "\n    return 0\n"
    scope = dict(ENV)
    exec(compile(source, "<loop IR>", "exec"), scope)
    fn, consts = scope["kernel"], list(py.consts)
    return lambda X, S: fn(X, S, consts)


def staged_ir(kernel, launch):
    """A staged kernel as plain loop IR: each item first copies its windows into local arrays of
    the windows' extents (``x{param}[base + c]`` for each ``c`` below the extent, every read
    bounds-checked, as the workgroup's copy into LDS reads them), then runs the item."""
    if not launch.stage:
        return kernel
    prefix = []
    for st in launch.stage:
        c = lir.Var("nc_c")
        prefix.append(lir.Array(st.name, st.extent, lir.Const(0.0 if st.dtype.name == "f32" else 0, st.dtype)))
        prefix.append(lir.Loop("nc_c", st.extent, (lir.ArrayStore(
            st.name, c, lir.Load(st.param, lir.Binary("add", st.base, c, lir.DType("i64")), st.dtype)),)))

    def wrap(stmts, depth):
        if depth == len(launch.grid):
            return tuple(prefix) + tuple(stmts)
        loop = stmts[0]
        return (lir.Loop(loop.var, loop.extent, wrap(loop.body, depth + 1), loop.kind),)

    return lir.Kernel(kernel.primitive, kernel.params, wrap(tuple(kernel.body), 0), kernel.bytes_read,
                      kernel.bytes_written)


def run(program, scheduled, inputs, weights, bound) -> dict:
    """Run ``program`` with its scheduled kernels [(kernel, Launch)] on the CPU; outputs by name.
    A staged launch runs as ``staged_ir`` writes it. A Fail returns ('fail', call index, code)."""
    fns = [compile_kernel(staged_ir(k, launch)) for k, launch in scheduled]
    store = {}
    for buf in program.buffers:
        shape = lir.shape_of(buf.shape, bound)
        if buf.kind == "input":
            store[buf] = np.ascontiguousarray(inputs[buf.name], buf.dtype.numpy).reshape(-1).copy()
        elif buf.kind == "weight":
            store[buf] = np.ascontiguousarray(weights[buf.name], buf.dtype.numpy).reshape(-1)
        elif buf.kind == "const":
            store[buf] = np.ascontiguousarray(buf.value, buf.dtype.numpy).reshape(-1)
        else:
            fill = np.nan if buf.dtype.name == "f32" else 0
            store[buf] = np.full(int(np.prod(shape, dtype=np.int64)), fill, buf.dtype.numpy)
    syms = [bound[s] for s in program.symbols]
    for c, call in enumerate(program.calls):
        kernel = scheduled[call.kernel][0]
        args = [store[call.output]]
        for i, view in enumerate(call.operands):
            param = kernel.params[i + 1]
            if param.packed is not None:
                rows, cols = view.buffer.shape
                args.append(pack_rows(store[view.buffer].reshape(rows, cols), param.packed).reshape(-1))
            else:
                args.append(store[view.buffer][lir.evaluate(view.offset, bound):])
        with np.errstate(all="ignore"):
            code = fns[call.kernel](args, syms)
        if code:
            return ("fail", c, code)
    return {name: store[buf].reshape(lir.shape_of(buf.shape, bound)) for name, buf in program.outputs.items()}


def bind(program, inputs) -> dict:
    bound = {}
    for name, _, shape in program.inputs:
        for d, n in zip(shape, np.asarray(inputs[name]).shape):
            sym = lir.as_symbol(d)
            if sym is not None and sym not in bound:
                bound[sym] = int(n)
    return bound


def schedules(program):
    """The GPU's default schedules for the program (what CompiledProgram builds)."""
    return gpu_schedule.schedule_program(program)
