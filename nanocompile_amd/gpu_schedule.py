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
* ``workgroup()``: one workgroup per item without a shared loop: every
  thread computes the item, thread 0 stores it (an item that only reads and
  reduces, given a workgroup so that its operands can be staged).
* ``stage(param)``: LDS staging. Every read of operand ``param`` in an item
  is ``base + v``, ``base`` fixed for the item and ``v`` one of the item's
  loops counting up to the same extent ``E``; the workgroup copies the
  window ``x[base, base + E)`` into LDS with coalesced loads once per item,
  and the reads go to LDS (a row read by every thread of a workgroup, or by
  one thread in order, leaves HBM once and at full width).
* ``lead()``: in a workgroup item, one wave computes the item's serial part
  (a row kernel's reductions before the shared loop, or a workgroup item's
  whole body) and the other waves wait at a barrier, then read the values the
  shared loop needs from LDS: the same values, computed once per workgroup
  instead of once per wave, so the waves no longer compete for issue slots
  with identical chains.
* ``hoist()``: with a lead wave, each serial loop of its part that updates
  one accumulator from one per-iteration value (the reference's reductions:
  ``acc = acc + t``, the NaN-propagating maximum over ``t``) has ``t``
  computed by every thread of the workgroup first, one iteration a thread,
  into LDS; the lead wave then runs the accumulator's chain over the stored
  values, in the loop's order. The values and the chain are the loop's own.
* ``lanes(array)``: an item's accumulator array of L independent chains (the
  reference's L accumulators, written one element per iteration of the
  innermost loops, whose indices enumerate 0..L-1) held one element per lane:
  an item becomes L lanes of a wavefront, lane l runs chain l (the loops that
  enumerated the chains become l's digits), and the statements after the
  chains read element i from lane i. Each chain is the same sequence of
  operations in the same order; only where it runs changes.
* ``vectorize(width)``: each thread takes ``width`` consecutive iterations of
  the loop spread across threads (the innermost grid loop, or the shared
  loop), so neighbouring reads and writes sit in one thread and can be
  issued as one wide access.
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

The space the autotuner searches mirrors the reference's (schedules.py:87-128:
per kernel class, the knobs and their values; the hand-written defaults;
``apply`` refusing a point outside the space): here the classes are ``row``
(an item ends in a loop its workgroup shares) and ``item`` (one thread per
item), and the knobs are the primitives above.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field, replace

from nanocompile_amd import lir, simplify

WAVE = 64
MAX_THREADS = 1024
MAX_STAGE_BYTES = 64 * 1024     # LDS a launch stages; a larger window at run time takes the unstaged kernel
VECTOR_WIDTHS = (1, 2, 4, 8)


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


def unconditional(x):
    """The nodes of ``x`` evaluated whenever ``x`` is: C evaluates one arm of ``?:`` and the
    right side of ``||`` only when the left is false."""
    yield x
    k = kind(x)
    if k == "Select":
        yield from unconditional(x.cond)
    elif k == "Binary" and x.op == "or":
        yield from unconditional(x.a)
    elif k in ("Load", "Local"):
        yield from unconditional(x.index)
    elif k == "Binary":
        yield from unconditional(x.a)
        yield from unconditional(x.b)
    elif k in ("Unary", "Cast"):
        yield from unconditional(x.a)
    elif k == "Fma":
        yield from unconditional(x.a)
        yield from unconditional(x.b)
        yield from unconditional(x.c)
    elif k == "Dp4":
        yield from unconditional(x.a)
        yield from unconditional(x.b)


def stmt_scalars(s) -> list:
    """The scalar expressions of one statement itself (not of the statements it holds)."""
    k = kind(s)
    if k == "Loop":
        return [s.extent]
    if k in ("Store", "ArrayStore"):
        return [s.index, s.value]
    if k in ("Let", "Assign"):
        return [s.value]
    if k == "Fail":
        return [s.cond]
    return []


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
class Staged:
    """An operand window copied into LDS once per item: ``x{param}[base, base + extent)``, read
    back as the local array ``name`` (``name[v]`` for the read ``x{param}[base + v]``)."""

    param: int
    name: str
    base: object                  # over the grid's loop vars, symbols and constants
    extent: object                # over symbols and constants: the same for every item
    dtype: object


@dataclass(frozen=True)
class Hoisted:
    """A serial loop of the lead wave's part (statement ``at`` of it) whose per-iteration value
    ``value`` (of dtype ``dtype``) every thread computes first into LDS array ``name`` (one
    element an iteration of ``var`` up to ``extent``); the accumulator's chain then reads it."""

    at: int
    var: str
    extent: object
    value: object                 # the expression stored (a Let's var, or the update's own operand)
    name: str
    dtype: object


@dataclass(frozen=True)
class Lanes:
    """Accumulator arrays of ``width`` elements held ``per_lane`` consecutive elements a lane:
    ``width / per_lane`` lanes an item; lane l runs the chains of elements l * per_lane + j,
    the chain loops' vars given by ``loops`` as (var, extent, coefficient), var = e /
    coefficient % extent for element e; ``index`` is the element index the chain statements use."""

    width: int
    arrays: tuple[str, ...]
    loops: tuple[tuple[str, int, int], ...]
    index: object
    per_lane: int = 1

    @property
    def lanes(self) -> int:
        """Lanes an item."""
        return self.width // self.per_lane


@dataclass(frozen=True)
class Launch:
    """How a scheduled kernel runs: its grid loops, workgroup size and the per-item mapping."""

    grid: tuple[str, ...] = ()
    threads: int = 256
    cooperate: str | None = None           # the loop shared by a workgroup's threads, one item per workgroup
    unroll: tuple[tuple[str, int], ...] = ()
    workgroup: bool = False                # one workgroup per item with no shared loop; thread 0 stores
    stage: tuple[Staged, ...] = ()         # operand windows staged in LDS per item
    vector: int = 1                        # consecutive iterations per thread of the loop spread across threads
    lead: bool = False                     # one wave computes the item's serial part, shared through LDS
    lanes: Lanes | None = None             # an item's accumulator arrays spread one element a lane
    hoist: tuple[Hoisted, ...] = ()        # lead-wave loops whose chain operands all threads compute first

    @property
    def per_workgroup(self) -> bool:
        """An item is a whole workgroup (else one thread)."""
        return self.cooperate is not None or self.workgroup

    def describe(self) -> str:
        parts = [f"grid({', '.join(self.grid)})", f"block({self.threads})"]
        if self.cooperate:
            parts.append(f"cooperate({self.cooperate})")
        if self.workgroup:
            parts.append("workgroup()")
        parts += [f"stage(x{st.param})" for st in self.stage]
        if self.lead:
            parts.append("lead()")
        if self.hoist:
            parts.append("hoist()")
        if self.lanes:
            per = f", {self.lanes.per_lane} a lane" if self.lanes.per_lane > 1 else ""
            parts.append(f"lanes({', '.join(self.lanes.arrays)}{per})")
        if self.vector > 1:
            parts.append(f"vectorize({self.vector})")
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
        if self.launch.workgroup:
            raise ScheduleError(f"cooperate({name}): the item is already a workgroup with no shared loop")
        self.launch = replace(self.launch, cooperate=name)
        self.steps.append(f"cooperate {name}")
        return self

    def workgroup(self) -> "GpuSchedule":
        """One workgroup per item with no loop shared: every thread computes the item, thread 0 stores."""
        if not self.launch.grid:
            raise ScheduleError("workgroup: bind the grid first")
        if self.launch.cooperate:
            raise ScheduleError("workgroup: the item already shares a loop across its workgroup")
        if self.launch.vector > 1:
            raise ScheduleError("workgroup: the item is vectorized across threads")
        self.launch = replace(self.launch, workgroup=True)
        self.steps.append("workgroup")
        return self

    def stage(self, param: int) -> "GpuSchedule":
        """Copy operand ``param``'s window into LDS once per item; its reads go to LDS.

        Legal when every read of the operand in the item is ``base + v``, with
        ``base`` the same for all of them and built from the grid's vars,
        symbols and constants, and ``v`` a loop var of the item whose loop
        counts to the same extent, itself built from symbols and constants;
        when one of the item's own loops counts to that extent and reads
        ``base + v`` in every iteration (so the unscheduled kernel reads every
        element of the window, and the copy reads nothing it would not); and
        when no ``Fail`` in the item can stop it before that loop.
        """
        launch = self.launch
        params = self.kernel.params
        if not launch.per_workgroup:
            raise ScheduleError(f"stage(x{param}): an item must be a workgroup (cooperate or workgroup) "
                                f"to share a staged window")
        if not 0 < param < len(params) or params[param].writable:
            raise ScheduleError(f"stage(x{param}): not an operand")
        if params[param].packed is not None:
            raise ScheduleError(f"stage(x{param}): read in a packed layout")
        if any(st.param == param for st in launch.stage):
            raise ScheduleError(f"stage(x{param}): already staged")
        body = self.item_body()
        if any(kind(x) == "Fail" for x in statements(body)):
            raise ScheduleError(f"stage(x{param}): the item checks its input and may stop before it has "
                                f"read the whole window")
        base, extent, reads = stage_window(body, param)
        itemsize = params[param].dtype.numpy.itemsize
        fixed = [st for st in launch.stage if kind(st.extent) == "Const"] + (
            [Staged(param, "", base, extent, params[param].dtype)] if kind(extent) == "Const" else [])
        if sum(_align16(int(st.extent.value) * st.dtype.numpy.itemsize) for st in fixed) > MAX_STAGE_BYTES:
            raise ScheduleError(f"stage(x{param}): {int(extent.value) * itemsize} bytes with the other windows "
                                f"exceed {MAX_STAGE_BYTES} bytes of LDS")
        name = f"nc_s{param}"
        dtype = params[param].dtype

        def rewrite(x):
            if kind(x) == "Load" and x.param == param:
                if x not in reads:
                    raise ScheduleError(f"stage(x{param}): read outside the item")
                return lir.Local(name, lir.Var(reads[x]), dtype)
            return x

        body = map_stmts(self.kernel.body, rewrite)
        self.kernel = lir.Kernel(self.kernel.primitive, tuple(params), body, self.kernel.bytes_read,
                                 self.kernel.bytes_written)
        self.launch = replace(launch, stage=launch.stage + (Staged(param, name, base, extent, dtype),))
        self.steps.append(f"stage x{param}")
        return self

    def lead(self) -> "GpuSchedule":
        """One wave computes the item's serial part; with a shared loop, the values it reads from
        that part reach the other waves through LDS after a barrier."""
        launch = self.launch
        if not launch.per_workgroup:
            raise ScheduleError("lead: an item must be a workgroup (cooperate or workgroup)")
        body = self.item_body()
        serial = body[:-1] if launch.cooperate else body
        if any(kind(x) == "Fail" for x in statements(serial)):
            # a failing wave returns; the others would wait at the barrier for it
            raise ScheduleError("lead: the serial part checks its input and may stop one wave early")
        if launch.cooperate and live_ins(body[:-1], body[-1]) is None:
            raise ScheduleError("lead: the shared loop reads an array the serial part fills")
        self.launch = replace(launch, lead=True)
        self.steps.append("lead")
        return self

    def hoist(self) -> "GpuSchedule":
        """Every hoistable loop of the lead wave's part (``hoistable``) gets its chain operand
        computed by all threads first; ScheduleError when none is."""
        launch = self.launch
        if not launch.lead:
            raise ScheduleError("hoist: needs a lead wave")
        body = self.item_body()
        serial = body[:-1] if launch.cooperate else body
        if any(kind(st) == "Array" for st in serial):
            # the phases split the lead wave's part into blocks; an array declared in one would
            # not be visible in the next
            raise ScheduleError("hoist: the lead wave's part declares an array")
        found = []
        staged = {st.name for st in launch.stage}
        for at, st in enumerate(serial):
            h = hoistable(serial, at, len(found), staged)
            if h is not None:
                found.append(h)
        if not found:
            raise ScheduleError("hoist: no loop of the lead wave's part updates one accumulator from one value")
        self.launch = replace(launch, hoist=tuple(found))
        self.steps.append("hoist")
        return self

    def lanes(self, name: str, per_lane: int = 1) -> "GpuSchedule":
        """Hold accumulator array ``name`` (and the arrays its chains update alongside it)
        ``per_lane`` consecutive elements a lane; see ``lane_chains`` for when that is legal.
        ``per_lane`` must divide the extent of the element index's unit digit (the innermost
        element loop), so a lane's elements differ in that digit alone: consecutive."""
        launch = self.launch
        if not launch.grid:
            raise ScheduleError("lanes: bind the grid first")
        if launch.per_workgroup or launch.vector > 1 or launch.lanes:
            raise ScheduleError("lanes: an item must be one thread's, not vectorized")
        lanes = lane_chains(self.item_body(), name)
        unit = next(extent for _, extent, coeff in lanes.loops if coeff == 1)
        if per_lane < 1 or per_lane & (per_lane - 1) or unit % per_lane:
            raise ScheduleError(f"lanes({name}, {per_lane}): not a power of two dividing the unit digit's {unit}")
        lanes = replace(lanes, per_lane=per_lane)
        if launch.threads % lanes.lanes:
            raise ScheduleError(f"lanes({name}): {lanes.lanes} lanes an item do not divide block({launch.threads})")
        self.launch = replace(launch, lanes=lanes)
        self.steps.append(f"lanes {name} {per_lane}")
        return self

    def vectorize(self, width: int) -> "GpuSchedule":
        """Each thread takes ``width`` consecutive iterations of the loop spread across threads."""
        if width not in VECTOR_WIDTHS:
            raise ScheduleError(f"vectorize({width}): one of {VECTOR_WIDTHS}")
        if not self.launch.grid:
            raise ScheduleError("vectorize: bind the grid first")
        if self.launch.workgroup:
            raise ScheduleError("vectorize: a workgroup item spreads no loop across its threads")
        if self.launch.lanes:
            raise ScheduleError("vectorize: the item's lanes hold its accumulators")
        self.launch = replace(self.launch, vector=width)
        self.steps.append(f"vectorize {width}")
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


# -- chains whose operands are computed first --------------------------------------------------


def hoistable(serial, at: int, k: int, staged=frozenset()) -> Hoisted | None:
    """Statement ``at`` of a lead wave's part as a Hoisted (its LDS array ``nc_h<k>``), when it is
    a loop whose body is Lets and then one update of an accumulator declared outside it, and
    the value the update takes each iteration is one expression free of the accumulator:
    either exactly one of the loop's Lets (the update reading it, the loop var and outer
    scalars), or, with no Lets, the other operand of ``acc op x``. The Lets and that value read
    no array but the ``staged`` windows (another thread would not have it), and the extent is
    the same for every item (symbols and constants), so the LDS array has one size."""
    loop = serial[at]
    if kind(loop) != "Loop" or not loop.body:
        return None
    *lets, update = loop.body
    if any(kind(s) != "Let" for s in lets) or kind(update) != "Assign":
        return None
    acc = update.var
    names = {s.var for s in lets}
    if acc in names or acc == loop.var:
        return None

    def private(x) -> bool:
        return any(kind(n) == "Local" and n.name not in staged for n in walk(x))

    if any(uses_var(s.value, acc) or private(s.value) for s in lets):
        return None
    if any(kind(n) in ("Var", "Load", "Local") for n in walk(loop.extent)):
        return None
    read = {n.name for n in walk(update.value) if kind(n) == "Var" and n.name in names}
    if lets:
        if len(read) != 1:
            return None
        name = read.pop()
        value = next(lir.Var(s.var, s.value.dtype) for s in lets if s.var == name)
    else:
        v = update.value
        if kind(v) != "Binary" or not any(kind(o) == "Var" and o.name == acc for o in (v.a, v.b)):
            return None
        value = v.b if kind(v.a) == "Var" and v.a.name == acc else v.a
        if uses_var(value, acc) or private(value) or kind(value) in ("Const", "Var"):
            return None
    return Hoisted(at, loop.var, loop.extent, value, f"nc_h{k}", value.dtype)


# -- accumulators across lanes ----------------------------------------------------------------


def _with_loops(stmts, loops=()):
    """Every statement with the loops around it (outermost first)."""
    for s in stmts:
        yield loops, s
        if kind(s) == "Loop":
            yield from _with_loops(s.body, loops + (s,))
        elif kind(s) == "Block":
            yield from _with_loops(s.body, loops)


def lane_chains(body, name: str) -> Lanes:
    """The Lanes for accumulator array ``name`` declared at the top of an item's ``body``, or
    ScheduleError. Legal when: the array's size L is a power of two from 2 to 64; every store
    to it (and to any array stored beside it) sits in one innermost nest of constant loops
    whose vars enumerate the element index e = sum(coefficient * var) over 0..L-1 exactly once
    (mixed radix), the nest holding only Lets and those stores; every read of those arrays in
    that nest is of element e (so each element's chain touches no other); nothing else in the
    item stores to them; and the item has no Fail (a lane that stopped would leave the others
    reading its element)."""
    arrays = {s.name: s for s in body if kind(s) == "Array"}
    if name not in arrays:
        raise ScheduleError(f"lanes({name}): no array {name} at the top of the item")
    width = int(arrays[name].size)
    if width < 2 or width > WAVE or width & (width - 1):
        raise ScheduleError(f"lanes({name}): {width} elements, not a power of two from 2 to {WAVE}")
    if any(kind(s) == "Fail" for s in statements(body)):
        raise ScheduleError(f"lanes({name}): the item checks its input and may stop early")
    stores = [(loops, s) for loops, s in _with_loops(body) if kind(s) == "ArrayStore" and s.name == name]
    if not stores:
        raise ScheduleError(f"lanes({name}): nothing stores to it")
    loops, first = stores[0]
    index = first.index
    a = simplify.affine(index)
    if a.const or not a.terms:
        raise ScheduleError(f"lanes({name}): the element index is not a sum of loop indices")
    by_var = {l.var: l for l in loops}
    digits = []
    for key, coeff in a.terms.items():
        atom = a.atoms[key]
        if kind(atom) != "Var" or atom.name not in by_var or coeff <= 0:
            raise ScheduleError(f"lanes({name}): the element index is not a sum of loop indices")
        loop = by_var[atom.name]
        if kind(loop.extent) != "Const":
            raise ScheduleError(f"lanes({name}): loop {loop.var} has no constant extent")
        digits.append((atom.name, int(loop.extent.value), int(coeff)))
    chain = list(loops[len(loops) - len(digits):])
    if sorted(l.var for l in chain) != sorted(v for v, _, _ in digits):
        raise ScheduleError(f"lanes({name}): the loops that enumerate the elements are not the innermost")
    for outer, inner in zip(chain, chain[1:]):
        if list(outer.body) != [inner]:
            raise ScheduleError(f"lanes({name}): the element loops are not perfectly nested")
    # the renderer maps a lane to its digits starting at the outermost loop of the nest, which
    # must therefore carry the largest coefficient, each inner loop a smaller one
    coefficient = {var: coeff for var, _, coeff in digits}
    nested = [coefficient[l.var] for l in chain]
    if any(outer <= inner for outer, inner in zip(nested, nested[1:])):
        raise ScheduleError(f"lanes({name}): the element loops are not nested from the largest "
                            f"coefficient inwards ({[l.var for l in chain]} have {nested})")
    radix = 1
    for var, extent, coeff in sorted(digits, key=lambda d: d[2]):
        if coeff != radix:
            raise ScheduleError(f"lanes({name}): the element index does not enumerate 0..{width - 1} once")
        radix *= extent
    if radix != width:
        raise ScheduleError(f"lanes({name}): the element loops enumerate {radix} elements, not {width}")
    inner_body = chain[-1].body
    group = set()
    for s in inner_body:
        if kind(s) == "Let":
            continue
        if kind(s) != "ArrayStore" or s.name not in arrays or int(arrays[s.name].size) != width or s.index != index:
            raise ScheduleError(f"lanes({name}): the chains do more than update elements {index!r}")
        group.add(s.name)
    for x in scalars(inner_body):
        if kind(x) == "Local" and (x.name in group or x.name in arrays) and (x.name not in group or x.index != index):
            raise ScheduleError(f"lanes({name}): a chain reads another element")
    for loops_of, s in _with_loops(body):
        if kind(s) == "ArrayStore" and s.name in group and s not in inner_body:
            raise ScheduleError(f"lanes({name}): {s.name} is stored outside its chains")
    return Lanes(width, tuple(sorted(group)), tuple(sorted(digits, key=lambda d: -d[2])), index)


# -- LDS staging -------------------------------------------------------------------------------


def live_ins(before, shared) -> list[tuple[str, object]] | None:
    """The scalars the shared loop reads that the statements before it declare (their top-level
    Lets, in order), with their types; None if it reads an array they declare."""
    used = set()
    for x in scalars((shared,)):
        for n in walk(x):
            if kind(n) == "Var":
                used.add(n.name)
            elif kind(n) == "Local":
                used.add(n.name)
    used |= {s.name for s in statements((shared,)) if kind(s) == "ArrayStore"}
    if any(kind(s) == "Array" and s.name in used for s in statements(before)):
        return None
    return [(s.var, s.value.dtype) for s in before if kind(s) == "Let" and s.var in used]


def _align16(n: int) -> int:
    return -(-int(n) // 16) * 16


def _split_read(index, loops: dict, local: set):
    """``index`` as ``(base, v)`` with ``index == base + v``, ``v`` one of ``loops``' vars and
    ``base`` free of item-local names and of loads; None when it is not of that form."""
    a = simplify.affine(index)
    hits = [k for k in a.terms if kind(a.atoms[k]) == "Var" and a.atoms[k].name in loops]
    if len(hits) != 1 or a.terms[hits[0]] != 1:
        return None
    rest = simplify.Affine(a.const, {k: c for k, c in a.terms.items() if k != hits[0]}, a.atoms)
    for k in rest.terms:
        for n in walk(rest.atoms[k]):
            if kind(n) in ("Load", "Local") or (kind(n) == "Var" and n.name in local):
                return None
    return simplify.expression(rest), a.atoms[hits[0]].name


def _reads_every_iteration(loop, param: int, base, loops: dict, local: set) -> bool:
    """Whether each iteration of ``loop`` reads ``x{param}[base + loop.var]`` unconditionally
    (in a statement of its own body, not of a nested loop, outside a lazily evaluated operand)."""
    pending = list(loop.body)
    while pending:
        st = pending.pop()
        if kind(st) == "Block":
            pending += list(st.body)
            continue
        if kind(st) == "Loop":
            continue
        for x in stmt_scalars(st):
            for n in unconditional(x):
                if kind(n) == "Load" and n.param == param:
                    split = _split_read(n.index, loops, local)
                    if split is not None and split[1] == loop.var and repr(split[0]) == repr(base):
                        return True
    return False


def stage_window(body, param: int) -> tuple:
    """(base, extent, {read: loop var}) of operand ``param``'s reads in an item's ``body``, or
    ScheduleError when they do not read one window that the item reads whole."""
    loops = {}
    for s in statements(body):
        if kind(s) == "Loop":
            if s.var in loops and repr(loops[s.var].extent) != repr(s.extent):
                raise ScheduleError(f"stage(x{param}): two loops {s.var} of the item count to different extents")
            loops[s.var] = s
    local = declared(body)
    reads = [x for x in scalars(body) if kind(x) == "Load" and x.param == param]
    if not reads:
        raise ScheduleError(f"stage(x{param}): the item does not read it")
    base = extent = None
    by_read = {}
    for x in reads:
        split = _split_read(x.index, loops, local)
        if split is None:
            raise ScheduleError(f"stage(x{param}): a read is not a base plus one of the item's loop indices")
        b, v = split
        e = loops[v].extent
        if any(kind(n) in ("Var", "Load", "Local") for n in walk(e)):
            raise ScheduleError(f"stage(x{param}): loop {v}'s extent changes from item to item")
        if base is None:
            base, extent = b, e
        elif repr(b) != repr(base) or repr(e) != repr(extent):
            raise ScheduleError(f"stage(x{param}): the reads span more than one window")
        by_read[x] = v
    top = [s for s in body if kind(s) == "Loop" and repr(s.extent) == repr(extent)]
    if not any(_reads_every_iteration(s, param, base, loops, local) for s in top):
        raise ScheduleError(f"stage(x{param}): no loop of the item reads the whole window")
    return base, extent, by_read


def unstage(kernel, launch) -> tuple:
    """The same kernel reading its staged operands from memory again and its lead wave computing
    its chains' operands itself: (kernel, launch without staging or hoisting); a launch whose
    LDS arrays do not fit at run time takes this kernel."""
    by_name = {st.name: st for st in launch.stage}

    def rewrite(x):
        if kind(x) == "Local" and x.name in by_name:
            st = by_name[x.name]
            return lir.Load(st.param, lir.Binary("add", st.base, x.index, I64), st.dtype)
        return x

    params = tuple(kernel.params)
    body = map_stmts(kernel.body, rewrite)
    return (lir.Kernel(kernel.primitive, params, body, kernel.bytes_read, kernel.bytes_written),
            replace(launch, stage=(), hoist=()))


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


def grid_loops(kernel) -> list[str]:
    """The outermost perfectly nested loops that can be the grid: independent, and each extent
    free of the loops outside it."""
    names = []
    for loop in perfect_nest(kernel.body):
        if not independent(loop) or any(uses_var(loop.extent, n) for n in names):
            break
        names.append(loop.var)
    return names


def shared_loop(kernel, names) -> str | None:
    """The loop a row kernel's workgroup shares: an item that ends in an independent loop that
    stores, after statements that only compute (reductions, then the write pass)."""
    if not names:
        return None
    body = tuple(perfect_nest(kernel.body)[len(names) - 1].body)
    last = body[-1] if body else None
    if (last is not None and kind(last) == "Loop" and len(body) > 1 and has_store((last,))
            and not has_store(body[:-1]) and independent(last)
            and not any(kind(x) == "Fail" for x in statements((last,)))):
        return last.var
    return None


# -- the space (schedules.py:87-128: SPACES, DEFAULTS, kernel_class, apply) ---------------------

# Each class's knobs and their values; the first value of each is the hand-written default's.
SPACES: dict[str, dict[str, tuple]] = {
    # a workgroup per item sharing its write pass: its size, its serial loops' operands staged in
    # LDS, iterations of the shared loop per thread, the serial loops' unroll (16, 64: their
    # operands read in batches of that many iterations ahead of the chain), one lead wave on the
    # serial part, its reductions' operands computed by every thread first
    "row": {"threads": (256, 64, 128, 512, 1024), "stage": (False, True), "vector": (1, 2, 4),
            "unroll": (0, 4, 16, 64), "lead": (False, True), "hoist": (False, True)},
    # a thread per item, or (workgroup) a workgroup per item with its loops' operands staged (a
    # lead wave, hoisting, as for rows), or (lanes) an item's accumulator chains 1 or 4 elements
    # a lane; weights packed in 64-row blocks or read row-major; serial loops unrolled up to 32
    # steps (a chain then reads that many steps' operands, in a batch, before its multiply-adds)
    "item": {"threads": (256, 64, 128, 512, 1024), "vector": (1, 2, 4), "workgroup": (False, True),
             "unroll": (0, 4, 16, 32), "lead": (False, True), "hoist": (False, True), "lanes": (0, 1, 4),
             "pack": (True, False)},
    # no loop can be the grid: one thread runs the kernel
    "serial": {"threads": (256,)},
}
DEFAULTS: dict[str, dict] = {cls: {k: v[0] for k, v in knobs.items()} for cls, knobs in SPACES.items()}


def kernel_class(kernel) -> str:
    names = grid_loops(kernel)
    if not names:
        return "serial"
    return "row" if shared_loop(kernel, names) else "item"


def canonical(config) -> tuple:
    """A hashable, order-independent form of ``config``."""
    return tuple(sorted(config.items()))


def space(kernel) -> list[dict]:
    """Every configuration of ``kernel``'s class, the default first, before asking which apply."""
    knobs = SPACES[kernel_class(kernel)]
    return [dict(zip(knobs, values)) for values in itertools.product(*knobs.values())]


_POINTS = {cls: {canonical(dict(zip(k, v))) for v in itertools.product(*k.values())} for cls, k in SPACES.items()}


def _serial_loops(s: "GpuSchedule") -> list[str]:
    """The item's loops one thread runs in order, long enough to unroll: an extent known to be at
    least 8 or set at run time, not the shared loop, neither reading nor storing a register
    array (loops over those are unrolled whole; an array held across lanes is a register or a
    few a lane and does not count), and not a loop that enumerates such an array's elements."""
    staged = {st.name for st in s.launch.stage}
    # arrays held across lanes are a register (or a few) a lane, indexed by nothing that varies;
    # the loops that enumerate their elements become the lane mapping
    held = set(s.launch.lanes.arrays) if s.launch.lanes else set()
    element_loops = {var for var, _, _ in s.launch.lanes.loops} if s.launch.lanes else set()
    out = []
    for st in statements(s.item_body()):
        if kind(st) != "Loop" or st.var == s.launch.cooperate or st.var in element_loops:
            continue
        if kind(st.extent) == "Const" and int(st.extent.value) < 8:
            continue
        arrays = any(kind(n) == "Local" and n.name not in staged and n.name not in held
                     for x in scalars(st.body) for n in walk(x))
        arrays = arrays or any(kind(t) == "ArrayStore" and t.name not in held for t in statements(st.body))
        if not arrays and st.var not in out:          # (two loops may share a name: one hint covers both)
            out.append(st.var)
    return out


def _reread_operands(s: "GpuSchedule") -> list[int]:
    """Operands the item reads inside a loop that one thread runs in order (each thread, or the one
    item thread, reads them element by element): the ones worth a copy in LDS."""
    out = []
    for st in statements(s.item_body()):
        if kind(st) != "Loop" or st.var == s.launch.cooperate:
            continue
        for x in scalars(st.body):
            if kind(x) == "Load" and x.param not in out:
                out.append(x.param)
    return sorted(out)


def _read_outside_hoisted(s: "GpuSchedule", param: int) -> bool:
    """Whether operand ``param`` is read by a statement of the item that hoisting ``s`` (a lead
    wave) leaves to the lead wave: outside every loop whose values all threads compute first.
    True when nothing can be hoisted (the lead wave then reads everything)."""
    trial = GpuSchedule(s.kernel, s.launch, list(s.steps))
    try:
        trial.lead().hoist()
    except ScheduleError:
        return True
    body = trial.item_body()
    serial = body[:-1] if trial.launch.cooperate else body
    hoisted = {h.at for h in trial.launch.hoist}
    rest = [st for at, st in enumerate(serial) if at not in hoisted] + list(body[len(serial):])
    return any(kind(x) == "Load" and x.param == param for x in scalars(tuple(rest)))


def apply(kernel, calls, config) -> tuple:
    """``kernel`` scheduled by ``config``: (kernel, Launch); ScheduleError if it does not apply.

    A configuration outside its class's space is an error, never rounded to a
    nearby point (schedules.py:187-197), and so is one whose knob has nothing
    to act on (staging with no operand to stage, unrolling with no serial
    loop), so each point of the space is a different kernel.
    """
    cls = kernel_class(kernel)
    config = dict(config)
    if canonical(config) not in _POINTS[cls]:
        raise ScheduleError(f"{config} is not a point of the {cls} space")
    s = GpuSchedule(kernel)
    names = grid_loops(kernel)
    if names:
        s.grid(*names)
    if cls == "row":
        s.cooperate(shared_loop(kernel, names))
    elif config.get("workgroup"):
        s.workgroup()
    s.block(config["threads"])
    if cls == "item" and config.get("pack", True):
        inner = names[-1]
        for param in range(1, len(kernel.params)):
            rc = _weight_rows(kernel, calls, param) if calls else None
            dp4 = any(kind(x) == "Dp4" and param in (x.a.param, x.b.param) for x in scalars(kernel.body))
            if rc and rc[0] >= WAVE and not dp4 and _reads_rows_by(kernel, param, inner, rc[1]):
                s.pack(param, rc[0], rc[1], WAVE)
    if config.get("stage") or config.get("workgroup"):
        operands = _reread_operands(s)
        # a workgroup item whose serial loops are all hoisted reads each operand once an element,
        # in the pass every thread runs: a copy in LDS would only add a pass and a barrier
        hoisted_only = cls == "item" and config.get("lead") and config.get("hoist")
        if hoisted_only:
            operands = [param for param in operands if _read_outside_hoisted(s, param)]
        for param in operands:
            try:
                s.stage(param)
            except ScheduleError:
                continue
        if not s.launch.stage and not hoisted_only:
            raise ScheduleError("no operand of the item can be staged")
    if config.get("lead"):
        s.lead()
    if config.get("hoist"):
        s.hoist()
    if config.get("lanes"):
        # lanes: elements a lane (0: one thread an item)
        arrays = [st.name for st in s.item_body() if kind(st) == "Array"]
        for name in arrays:
            try:
                s.lanes(name, int(config["lanes"]))
                break
            except ScheduleError:
                continue
        if not s.launch.lanes:
            raise ScheduleError("no accumulator array of the item can be spread over lanes")
    if config.get("vector", 1) > 1:
        s.vectorize(config["vector"])
    if config.get("unroll"):
        loops = _serial_loops(s)
        if not loops:
            raise ScheduleError("no serial loop to unroll")
        for var in loops:
            s.unroll(var, config["unroll"])
    return s.done()


def _reduces_over_run_time_extent(kernel) -> bool:
    """Whether the item runs a serial loop whose extent is set at run time (a symbol): a reduction
    as long as the context, like attention's P.V over past + seq positions."""
    grid = set(grid_loops(kernel))
    for st in statements(kernel.body):
        if kind(st) == "Loop" and st.var not in grid and any(kind(n) == "Sym" for n in walk(st.extent)):
            return True
    return False


# The default schedule of each class: the first of these points that applies to the kernel. They
# are what the tuner chose on the reference's own programs (config 5's decode step, the zoo) on
# MI355X, most specific first, each falling back to the next where a knob has nothing to act on,
# and last the space's base point, which applies to every kernel of its class.
PREFERRED: dict[str, tuple] = {
    "item": (
        # int8 projections: the 32 accumulator chains one a lane, the weights read row-major so an
        # item's lanes read consecutive bytes, the k loop unrolled so its loads issue ahead
        dict(DEFAULTS["item"], threads=64, lanes=1, pack=False, unroll=16),
        dict(DEFAULTS["item"], threads=64, lanes=1, pack=False),
        # a reduction as long as the context (P.V): a workgroup an item, its operands staged and
        # computed by every thread, one wave on the chain
        ("run-time reduction", dict(DEFAULTS["item"], threads=128, workgroup=True, lead=True, hoist=True,
                                    unroll=16)),
        ("run-time reduction", dict(DEFAULTS["item"], threads=128, workgroup=True, lead=True)),
        # anything else with a serial loop: unrolled, small blocks
        dict(DEFAULTS["item"], threads=64, unroll=16),
        DEFAULTS["item"],
    ),
    "row": (
        # a reduction of fixed length (rms_norm's sum of squares over the hidden size): one lead
        # wave on it, its operands computed by every thread first (hoisted) and read back in
        # batches of 64 ahead of the chain
        ("fixed-length reduction", dict(DEFAULTS["row"], threads=512, vector=4, unroll=64, lead=True, hoist=True)),
        # one over a run-time length (softmax's sums over the context): the same, the row read from
        # HBM by each pass (no staging) and the chain's operands read back in batches of 16
        ("run-time reduction", dict(DEFAULTS["row"], threads=512, unroll=16, lead=True, hoist=True)),
        # row kernels: one lead wave on the row's reductions, their operands computed by every
        # thread first (hoisted), the row staged in LDS
        dict(DEFAULTS["row"], threads=512, stage=True, lead=True, hoist=True),
        dict(DEFAULTS["row"], threads=1024, lead=True, hoist=True, vector=4),
        dict(DEFAULTS["row"], threads=512, lead=True, hoist=True),
        dict(DEFAULTS["row"], threads=1024, stage=True, lead=True, vector=4),
        dict(DEFAULTS["row"], threads=512, lead=True),
        DEFAULTS["row"],
    ),
    "serial": (DEFAULTS["serial"],),
}


def default_config(kernel, calls=()) -> dict:
    """The point of ``kernel``'s space that its default schedule is (``PREFERRED``)."""
    run_time = None
    for entry in PREFERRED[kernel_class(kernel)]:
        if isinstance(entry, tuple):
            if run_time is None:
                run_time = _reduces_over_run_time_extent(kernel)
            if run_time != (entry[0] == "run-time reduction"):
                continue
            entry = entry[1]
        try:
            apply(kernel, calls, entry)
        except ScheduleError:
            continue
        return dict(entry)
    raise ScheduleError(f"no default applies to this {kernel_class(kernel)} kernel")


def default(kernel, calls=()) -> tuple:
    """The library's schedule for a kernel: (scheduled kernel, Launch).

    Every top-level independent loop binds to the grid. An item whose body
    ends in an independent loop that stores, after statements that only
    compute (a row kernel: reductions, then the write pass), runs as one
    workgroup per item with the write pass across its threads, one wave on
    its reductions. Otherwise an item is a thread, its int8 accumulators
    spread over lanes where it has them, or (a reduction over the context) a
    workgroup; weights an item reads row by row are packed in blocks of 64
    rows, except where lanes read them row-major. ``default_config`` names the
    point; ``DEFAULTS`` is the space's base point, which applies everywhere.
    """
    return apply(kernel, calls, default_config(kernel, calls))


def schedule_program(program, fn=default):
    """Each distinct kernel scheduled once, with the calls that run it: [(kernel, Launch)]."""
    calls_of: dict[int, list] = {}
    for call in program.calls:
        calls_of.setdefault(call.kernel, []).append(call)
    return [fn(k, calls_of.get(i, [])) for i, k in enumerate(program.kernels)]
