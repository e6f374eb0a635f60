"""GPU schedules: how a loop-IR kernel's iterations map onto a gfx950 launch.

The reference schedules a kernel for the CPU by rewriting its loop nest
(schedule.py: split, reorder, unroll, privatize, vectorize, parallel, pack),
each transformation checked for legality and none reordering the operations
that produce a value, so a scheduled kernel is bitwise the kernel it came
from (schedule.py:14-19). The same rule holds here; what changes is the
space. A GPU launch binds loops to the grid instead of to a thread pool:

* ``grid(vars)``: the kernel's outermost perfectly nested loops, iterations
  independent, become the launch's items (flattened, the last var fastest).
* ``block(threads)``: workgroup size, a multiple of the 64-lane wavefront.
* ``cooperate(var)``: one workgroup per item instead of one thread: the
  item's statements before loop ``var`` (its reductions, which only compute
  item-local values) run in every thread of the workgroup, each thread
  computing the same value in the same order, and ``var``'s independent
  iterations are shared among the threads (a row kernel's write pass across
  a workgroup, with its sums computed once per thread, in order).
* ``unroll(var, factor)``: a constant-count unroll hint for a serial loop.
* ``pack(param, rows, cols, block)``: the reference's packed operand layout
  (schedule.py:362-395, loopir.Param.packed): rows in blocks of ``block``,
  column-major within a block, so that with 64 rows a block the 64 lanes of
  a wavefront walking consecutive rows read 64 consecutive elements at each
  step of their own k loops: coalesced, where row-major rows are strided.
  Rows need not be a multiple of ``block`` here: the runtime pads the packed
  copy, and the reads of real rows are unchanged.

None of these changes an arithmetic operation or its order: each output
element is computed by the same expression sequence as in the unscheduled
kernel, so every schedule is bitwise the unscheduled kernel, and the tests
and the autotuner hold every candidate to that.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace

from nanocompile_amd import lir

WAVE = 64
MAX_THREADS = 1024


class ScheduleError(ValueError):
    """A GPU schedule that does not apply to the kernel, or would change what it computes."""


def kind(x) -> str:
    return type(x).__name__


# -- what a loop nest reads and writes ------------------------------------------------------


def declared(stmts) -> set[str]:
    out: set[str] = set()
    for s in stmts:
        k = kind(s)
        if k == "Loop":
            out.add(s.var)
            out |= declared(s.body)
        elif k == "Block":
            out |= declared(s.body)
        elif k == "Let":
            out.add(s.var)
        elif k == "Array":
            out.add(s.name)
    return out


def written(stmts) -> set[str]:
    out: set[str] = set()
    for s in stmts:
        k = kind(s)
        if k in ("Loop", "Block"):
            out |= written(s.body)
        elif k == "Assign":
            out.add(s.var)
        elif k == "ArrayStore":
            out.add(s.name)
    return out


def independent(loop) -> bool:
    """No iteration updates a scalar or array declared outside the loop (stores to the output do not count)."""
    return not (written(loop.body) - declared(loop.body))


def walk(x):
    """A scalar node and every node below it."""
    yield x
    k = kind(x)
    if k in ("Load", "Local"):
        yield from walk(x.index)
    elif k == "Binary":
        yield from walk(x.a)
        yield from walk(x.b)
    elif k in ("Unary", "Cast"):
        yield from walk(x.a)
    elif k == "Select":
        yield from walk(x.cond)
        yield from walk(x.a)
        yield from walk(x.b)
    elif k == "Fma":
        yield from walk(x.a)
        yield from walk(x.b)
        yield from walk(x.c)
    elif k == "Dp4":
        yield from walk(x.a)
        yield from walk(x.b)


def scalars(stmts):
    for s in stmts:
        k = kind(s)
        if k == "Loop":
            yield from walk(s.extent)
            yield from scalars(s.body)
        elif k == "Block":
            yield from scalars(s.body)
        elif k in ("Store", "ArrayStore"):
            yield from walk(s.index)
            yield from walk(s.value)
        elif k in ("Let", "Assign"):
            yield from walk(s.value)
        elif k == "Fail":
            yield from walk(s.cond)


def statements(stmts):
    for s in stmts:
        yield s
        if kind(s) in ("Loop", "Block"):
            yield from statements(s.body)


def uses_var(x, name: str) -> bool:
    return any(kind(n) == "Var" and n.name == name for n in walk(x))


def has_store(stmts) -> bool:
    return any(kind(s) == "Store" for s in statements(stmts))


def perfect_nest(body) -> list:
    """The chain of loops at the top of ``body`` each holding only the next: [L1, L2, ...]."""
    chain = []
    stmts = body
    while len(stmts) == 1 and kind(stmts[0]) == "Loop":
        chain.append(stmts[0])
        stmts = stmts[0].body
    return chain


# -- rewriting loads (pack) ----------------------------------------------------------------


def _map_scalar(x, f):
    k = kind(x)
    if k == "Load":
        x = lir.Load(x.param, _map_scalar(x.index, f), x.dtype)
    elif k == "Local":
        x = lir.Local(x.name, _map_scalar(x.index, f), x.dtype)
    elif k == "Binary":
        x = lir.Binary(x.op, _map_scalar(x.a, f), _map_scalar(x.b, f), x.dtype)
    elif k == "Unary":
        x = lir.Unary(x.op, _map_scalar(x.a, f), x.dtype)
    elif k == "Select":
        x = lir.Select(_map_scalar(x.cond, f), _map_scalar(x.a, f), _map_scalar(x.b, f), x.dtype)
    elif k == "Cast":
        x = lir.Cast(_map_scalar(x.a, f), x.dtype)
    elif k == "Fma":
        x = lir.Fma(_map_scalar(x.a, f), _map_scalar(x.b, f), _map_scalar(x.c, f), x.dtype)
    elif k == "Dp4":
        x = lir.Dp4(_map_scalar(x.a, f), _map_scalar(x.b, f), x.dtype)
    return f(x)


def map_stmts(stmts, f) -> tuple:
    out = []
    for s in stmts:
        k = kind(s)
        if k == "Loop":
            out.append(lir.Loop(s.var, _map_scalar(s.extent, f), map_stmts(s.body, f), s.kind))
        elif k == "Block":
            out.append(lir.Block(map_stmts(s.body, f)))
        elif k == "Store":
            out.append(lir.Store(s.param, _map_scalar(s.index, f), _map_scalar(s.value, f)))
        elif k == "Let":
            out.append(lir.Let(s.var, _map_scalar(s.value, f)))
        elif k == "Assign":
            out.append(lir.Assign(s.var, _map_scalar(s.value, f)))
        elif k == "Fail":
            out.append(lir.Fail(_map_scalar(s.cond, f), s.code))
        elif k == "ArrayStore":
            out.append(lir.ArrayStore(s.name, _map_scalar(s.index, f), _map_scalar(s.value, f)))
        else:
            out.append(s)
    return tuple(out)


I64 = lir.DType("i64")


def _c(v: int):
    return lir.Const(v, I64)


# -- the schedule -------------------------------------------------------------------------------


@dataclass(frozen=True)
class Launch:
    """How a scheduled kernel runs: its grid loops, workgroup size and the per-item mapping."""

    grid: tuple[str, ...] = ()
    threads: int = 256
    cooperate: str | None = None           # the loop shared by a workgroup's threads, one item per workgroup
    unroll: tuple[tuple[str, int], ...] = ()

    def describe(self) -> str:
        parts = [f"grid({', '.join(self.grid)})", f"block({self.threads})"]
        if self.cooperate:
            parts.append(f"cooperate({self.cooperate})")
        parts += [f"unroll({v}, {n})" for v, n in self.unroll]
        return ".".join(parts)


@dataclass
class GpuSchedule:
    """A kernel being scheduled for the GPU; each method applies one primitive and checks it."""

    kernel: object
    launch: Launch = field(default_factory=Launch)
    steps: list = field(default_factory=list)

    @property
    def nest(self) -> list:
        return perfect_nest(self.kernel.body)

    def grid(self, *names: str) -> "GpuSchedule":
        nest = self.nest
        if len(names) > len(nest) or [l.var for l in nest[:len(names)]] != list(names):
            raise ScheduleError(f"grid{names}: not the kernel's outermost perfectly nested loops "
                                f"({[l.var for l in nest]})")
        for loop in nest[:len(names)]:
            if not independent(loop):
                raise ScheduleError(f"grid: an iteration of {loop.var} carries a value into the next")
            for outer in names:
                if uses_var(loop.extent, outer):
                    raise ScheduleError(f"grid: {loop.var}'s extent depends on {outer}")
        self.launch = replace(self.launch, grid=tuple(names))
        self.steps.append(f"grid {' '.join(names)}")
        return self

    def block(self, threads: int) -> "GpuSchedule":
        if threads <= 0 or threads % WAVE or threads > MAX_THREADS:
            raise ScheduleError(f"block({threads}): a multiple of {WAVE} up to {MAX_THREADS}")
        self.launch = replace(self.launch, threads=threads)
        self.steps.append(f"block {threads}")
        return self

    def item_body(self) -> tuple:
        grid = self.launch.grid
        if not grid:
            return tuple(self.kernel.body)
        return tuple(self.nest[len(grid) - 1].body)

    def cooperate(self, name: str) -> "GpuSchedule":
        if not self.launch.grid:
            raise ScheduleError("cooperate: bind the grid first")
        body = self.item_body()
        at = [i for i, s in enumerate(body) if kind(s) == "Loop" and s.var == name]
        if not at:
            raise ScheduleError(f"cooperate({name}): no loop {name} directly in the item's body")
        i = at[-1]
        loop, before, after = body[i], body[:i], body[i + 1:]
        if has_store(before):
            raise ScheduleError(f"cooperate({name}): the statements before it store to the output, "
                                f"which every thread would repeat")
        if after:
            raise ScheduleError(f"cooperate({name}): statements follow the loop")
        if not independent(loop):
            raise ScheduleError(f"cooperate({name}): an iteration carries a value into the next")
        if any(kind(s) == "Fail" for s in statements(loop.body)):
            raise ScheduleError(f"cooperate({name}): the loop checks its input and may stop early")
        self.launch = replace(self.launch, cooperate=name)
        self.steps.append(f"cooperate {name}")
        return self

    def unroll(self, name: str, factor: int) -> "GpuSchedule":
        loops = [s for s in statements(self.kernel.body) if kind(s) == "Loop" and s.var == name]
        if not loops:
            raise ScheduleError(f"unroll({name}): no such loop")
        if factor < 1:
            raise ScheduleError(f"unroll({name}, {factor}): the factor must be positive")
        self.launch = replace(self.launch, unroll=self.launch.unroll + ((name, factor),))
        self.steps.append(f"unroll {name} {factor}")
        return self

    def pack(self, param: int, rows: int, cols: int, block: int = WAVE) -> "GpuSchedule":
        params = list(self.kernel.params)
        if not 0 < param < len(params) or params[param].writable:
            raise ScheduleError(f"pack(x{param}): not an operand")
        if params[param].packed is not None:
            raise ScheduleError(f"pack(x{param}): already packed")
        if rows <= 0 or cols <= 0 or block <= 0:
            raise ScheduleError(f"pack(x{param}): bad shape [{rows}, {cols}] / {block}")
        if any(kind(x) == "Dp4" and param in (x.a.param, x.b.param) for x in scalars(self.kernel.body)):
            # a Dp4 reads four consecutive elements from its address, which packing separates
            raise ScheduleError(f"pack(x{param}): a Dp4 reads it four elements at a time")

        def rewrite(x):
            if kind(x) == "Load" and x.param == param:
                flat = x.index
                row = lir.Binary("idiv", flat, _c(cols), I64)
                col = lir.Binary("mod", flat, _c(cols), I64)
                index = lir.Binary("add", lir.Binary("add", lir.Binary("mul", lir.Binary("idiv", row, _c(block), I64),
                                                                             _c(cols * block), I64),
                                                     lir.Binary("mul", col, _c(block), I64), I64),
                                   lir.Binary("mod", row, _c(block), I64), I64)
                return lir.Load(param, index, x.dtype)
            return x

        params[param] = lir.Param(params[param].dtype, params[param].writable, block)
        body = map_stmts(self.kernel.body, rewrite)
        self.kernel = lir.Kernel(self.kernel.primitive, tuple(params), body, self.kernel.bytes_read,
                                 self.kernel.bytes_written)
        self.steps.append(f"pack x{param} {rows}x{cols}/{block}")
        return self

    def done(self) -> tuple:
        from nanocompile_amd import simplify
        kernel = lir.Kernel(self.kernel.primitive, tuple(self.kernel.params), simplify.simplify_body(self.kernel.body),
                            self.kernel.bytes_read, self.kernel.bytes_written)
        return kernel, self.launch


# -- the default schedule ----------------------------------------------------------------


def _weight_rows(kernel, calls, param: int):
    """[rows, cols] of operand ``param`` when every call hands it a whole row-major 2-D weight."""
    shapes = set()
    for call in calls:
        view = call.operands[param - 1]
        buf = view.buffer
        if buf.kind != "weight" or len(buf.shape) != 2 or not all(isinstance(d, int) for d in buf.shape):
            return None
        if not isinstance(view.offset, int) or view.offset != 0:
            return None
        shapes.add(tuple(buf.shape))
    return shapes.pop() if len(shapes) == 1 else None


def _reads_rows_by(kernel, param: int, var: str, cols: int) -> bool:
    """Every load of ``param`` reads ``var * cols + (something not using var)``: each value of the
    innermost grid var walks its own row of the operand."""
    from nanocompile_amd import simplify
    loads = [x for x in scalars(kernel.body) if kind(x) == "Load" and x.param == param]
    if not loads:
        return False
    return all(simplify.coefficient(x.index, var) == cols for x in loads)


def default(kernel, calls=()) -> tuple:
    """The library's schedule for a kernel: (scheduled kernel, Launch).

    Every top-level independent loop binds to the grid. An item whose body
    ends in an independent loop that stores, after statements that only
    compute (a row kernel: reductions, then the write pass), runs as one
    workgroup per item with the write pass across its threads. Otherwise one
    thread per item; weights read row by row by consecutive items are packed
    in blocks of 64 rows so a wavefront's reads coalesce.
    """
    s = GpuSchedule(kernel)
    nest = perfect_nest(kernel.body)
    names = []
    for loop in nest:
        if not independent(loop) or any(uses_var(loop.extent, n) for n in names):
            break
        names.append(loop.var)
    if names:
        s.grid(*names)
    body = s.item_body()
    last = body[-1] if body else None
    if (names and last is not None and kind(last) == "Loop" and len(body) > 1 and has_store((last,))
            and not has_store(body[:-1]) and independent(last)
            and not any(kind(x) == "Fail" for x in statements((last,)))):
        s.cooperate(last.var)
        s.block(256)
        return s.done()
    s.block(256)
    if names:
        inner = names[-1]
        for param in range(1, len(kernel.params)):
            rc = _weight_rows(kernel, calls, param) if calls else None
            dp4 = any(kind(x) == "Dp4" and param in (x.a.param, x.b.param) for x in scalars(kernel.body))
            if rc and rc[0] >= WAVE and not dp4 and _reads_rows_by(kernel, param, inner, rc[1]):
                s.pack(param, rc[0], rc[1], WAVE)
    return s.done()


def schedule_program(program, fn=default):
    """Each distinct kernel scheduled once, with the calls that run it: [(kernel, Launch)]."""
    calls_of: dict[int, list] = {}
    for call in program.calls:
        calls_of.setdefault(call.kernel, []).append(call)
    return [fn(k, calls_of.get(i, [])) for i, k in enumerate(program.kernels)]
