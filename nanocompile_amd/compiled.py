"""Running a compiled program on the GPU: one device arena, a liveness plan per call, the launch loop.

This is the reference's compile-then-call runtime (runtime.py:167-301) with
the C library replaced by a HIP one (codegen_hip.py):

* **Compile**: each distinct kernel gets a GPU schedule (gpu_schedule.py, or
  a tuner's choice), the library is rendered and built through the
  content-addressed cache, loaded, and bound to the package's stream and
  error word (``nc_bind_stream``, where the reference binds its thread pool).
* **Memory**: one ``hipMalloc`` arena. Its first region holds the weights
  and constants, uploaded once per weights mapping (and once per packed
  layout a schedule asks for); the rest holds a call's inputs, outputs and
  temporaries. Temporaries share space by a best-fit plan over the calls in
  order, made per call because sizes depend on ``seq`` and ``past``: a call's
  output block is taken before the blocks whose last reader it is are given
  back, so no kernel ever writes one of its own operands (runtime.py:1-14
  states the same rule for its host arena). A call needing more room than
  the arena has grows it, the weights moved over by one device copy.
* **Calls**: each kernel's launcher gets its output and operand device
  pointers (each operand's view offset applied) and the symbol values, in
  the reference's ``int32_t f(void **p, const int64_t *s)`` convention. The
  launches are queued back to back on one stream; the host waits once, at
  the end, then reads the error word: a kernel's ``Fail`` becomes the
  reference's KernelError, naming the gather that failed and its bad index
  (runtime.py:303-318).
"""

from __future__ import annotations

import ctypes
import time
from collections.abc import Mapping
from dataclasses import dataclass

import numpy as np

from nanocompile_amd import codegen_hip, gpu_schedule, hip, lir
from nanocompile_amd.hip import KernelError

ALIGN = 256
KERNEL_TYPE = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64))


class ArgumentError(ValueError):
    """Inputs or weights that do not match the graph's interface."""


def _align(n: int) -> int:
    return -(-max(int(n), 1) // ALIGN) * ALIGN


def _nbytes(buf, bound) -> int:
    return int(np.prod(lir.shape_of(buf.shape, bound), dtype=np.int64)) * buf.dtype.numpy.itemsize


# -- the plan ----------------------------------------------------------------------------------


@dataclass(frozen=True)
class Plan:
    offsets: dict                 # temp buffer -> byte offset in the call region
    region_bytes: int             # the temporaries' region
    unshared_bytes: int           # what they would take with no reuse


def plan_memory(program, last_use: Mapping, bound: Mapping[str, int]) -> Plan:
    """Temporaries placed in call order: each output in the smallest free block that holds it
    (else at the top), then the blocks whose last reader this call is freed and merged."""
    dying: dict[int, list] = {}
    for buf, index in last_use.items():
        dying.setdefault(index, []).append(buf)
    free: list[list[int]] = []                 # [offset, size], kept sorted and merged
    top = 0
    offsets, sizes = {}, {}
    unshared = 0
    for index, call in enumerate(program.calls):
        out = call.output
        if out.kind == "temp" and out not in offsets:
            size = _align(_nbytes(out, bound))
            fits = [i for i, (_, block) in enumerate(free) if block >= size]
            if fits:
                i = min(fits, key=lambda j: (free[j][1], free[j][0]))
                at, block = free.pop(i)
                if block > size:
                    free.append([at + size, block - size])
                    free.sort()
            else:
                at, top = top, top + size
            offsets[out], sizes[out] = at, size
            unshared += size
        for buf in dying.get(index, ()):
            if buf not in offsets:
                continue
            free.append([offsets[buf], sizes[buf]])
            free.sort()
            merged: list[list[int]] = []
            for at, block in free:
                if merged and merged[-1][0] + merged[-1][1] == at:
                    merged[-1][1] += block
                else:
                    merged.append([at, block])
            free = merged
    return Plan(offsets, top, unshared)


@dataclass(frozen=True)
class Layout:
    """Where one call's buffers sit in the arena's call region (byte offsets from its start)."""

    offsets: dict                 # input, output and temp buffers -> offset
    sizes: dict                   # the same buffers -> bytes reserved
    bytes: int                    # the call region's size


def call_layout(program, bound: Mapping[str, int], plan: Plan) -> Layout:
    """Inputs, then outputs, then the temporaries' plan: each input and output its own block."""
    offsets, sizes, at = {}, {}, 0
    for buf in program.buffers:
        if buf.kind in ("input", "output"):
            size = _align(_nbytes(buf, bound))
            offsets[buf], sizes[buf], at = at, size, at + size
    for buf, offset in plan.offsets.items():
        offsets[buf] = at + offset
        sizes[buf] = _align(_nbytes(buf, bound))
    return Layout(offsets, sizes, at + plan.region_bytes)


def schedule_of(program, schedule="default") -> list:
    """[(scheduled kernel, Launch)] for each distinct kernel of ``program``."""
    if schedule == "default":
        return gpu_schedule.schedule_program(program)
    if hasattr(schedule, "schedule_program"):
        return schedule.schedule_program(program)
    return gpu_schedule.schedule_program(program, schedule)


def prebuild(program, schedule_fn="default"):
    """Render and build ``program``'s library into the cache without touching a GPU: (path, cached)."""
    program = lir.adapt(program)
    return codegen_hip.build_library(codegen_hip.render_library(schedule_of(program, schedule_fn)))


def pack_rows(source: np.ndarray, block: int) -> np.ndarray:
    """A row-major [rows, cols] array in the packed layout (loopir.Param.packed, schedule.py:362-395):
    element (r, c) at (r / block) * cols * block + c * block + r % block, rows padded to whole blocks."""
    rows, cols = source.shape
    padded = -(-rows // block) * block
    out = np.zeros((padded, cols), source.dtype)
    out[:rows] = source
    return np.ascontiguousarray(out.reshape(padded // block, block, cols).transpose(0, 2, 1))


# -- the compiled program -------------------------------------------------------------------------


class CompiledProgram:
    """A program lowered to HIP, built, loaded, and callable like the reference's CompiledGraph.

    ``program`` is the reference's Program (fusion.fuse's result) or this
    package's reading of one (``lir.program_from_json``). ``schedule`` is
    ``"default"`` (gpu_schedule.default), a function ``(kernel, calls) ->
    (kernel, Launch)``, an object with ``schedule_program(program)``, or one
    with ``library_for(program)`` returning ``(scheduled, source, launcher
    names)``: a library that holds the chosen kernels among others (the
    autotuner's, whose candidates were measured in that same library).
    """

    def __init__(self, program, schedule="default", device: int = 0) -> None:
        started = time.perf_counter()
        hip.init(device)
        program = lir.adapt(program)
        self.program = program
        if hasattr(schedule, "library_for"):
            self.scheduled, self.source, names = schedule.library_for(program)
        else:
            self.scheduled = schedule_of(program, schedule)
            self.source = codegen_hip.render_library(self.scheduled)
            names = [codegen_hip.kernel_name(i) for i in range(len(self.scheduled))]
        self.kernels = [k for k, _ in self.scheduled]
        self.library_path, self.cached = codegen_hip.build_library(self.source)
        self.compile_seconds = time.perf_counter() - started
        self._library = ctypes.CDLL(str(self.library_path))
        bind = self._library.nc_bind_stream
        bind.argtypes, bind.restype = [ctypes.c_void_p, ctypes.c_void_p], None
        bind(hip.load().nc_stream_handle(), hip.load().nc_error_word())
        self.launcher_names = list(names)
        self._launch = [KERNEL_TYPE((name, self._library)) for name in names]
        self._last_use = program.last_uses()
        self.symbols = tuple(program.symbols)
        # operands read in a packed layout: (call, operand) -> rows per block
        self._packed = {(c, i): self.kernels[call.kernel].params[i + 1].packed
                        for c, call in enumerate(program.calls)
                        for i in range(len(call.operands))
                        if self.kernels[call.kernel].params[i + 1].packed is not None}
        # a packed copy is made once, at upload, so it must cover a whole matrix that never changes
        for (c, i), block in self._packed.items():
            operand = program.calls[c].operands[i]
            buf = operand.buffer
            if not (buf.kind == "weight" and len(buf.shape) == 2 and operand.offset == 0):
                raise ValueError(f"packed operand {i} of call {c} is {buf!r}: a packed layout is made "
                                 f"for an unsliced two-dimensional weight and nothing else")
        self._arena: hip.DeviceArray | None = None
        self._resident: dict = {}          # (buffer name or id, packing) -> offset in the weight region
        self._held: dict | None = None     # name -> the very array uploaded (kept alive, compared by identity)
        self._region = 0                   # bytes of the weight region
        self.last_plan: Plan | None = None

    # -- arguments --------------------------------------------------------------------------

    def bind(self, inputs: Mapping[str, np.ndarray], weights: Mapping[str, np.ndarray],
             bindings: Mapping[str, int] | None = None) -> dict[str, int]:
        """Check a call's arguments against the graph's interface; the symbols' values."""
        names = [name for name, _, _ in self.program.inputs]
        unknown, missing = sorted(set(inputs) - set(names)), sorted(set(names) - set(inputs))
        if unknown or missing:
            raise ArgumentError(f"inputs: missing {missing}, unexpected {unknown}")
        bound: dict[str, int] = {}
        for name, _, shape in self.program.inputs:
            array = np.asarray(inputs[name])
            if array.ndim != len(shape):
                raise ArgumentError(f"input {name!r} has {array.ndim} dimensions, expected {len(shape)}")
            for d, n in zip(shape, array.shape):
                symbol = lir.as_symbol(d)
                if symbol is not None and symbol not in bound:
                    bound[symbol] = int(n)
        for name, value in (bindings or {}).items():
            if name in bound and bound[name] != int(value):
                raise ArgumentError(f"binding {name}={value} disagrees with the inputs ({name}={bound[name]})")
            bound[name] = int(value)
        for name, dtype, shape in self.program.inputs:
            array = np.asarray(inputs[name])
            want = lir.shape_of(shape, bound)
            if array.dtype != dtype.numpy or tuple(array.shape) != want:
                raise ArgumentError(f"input {name!r} is {array.dtype}{list(array.shape)}, expected "
                                    f"{dtype.name}{list(want)}")
        for name, (dtype, shape) in self.program.weights.items():
            if name not in weights:
                raise ArgumentError(f"weight {name!r} is missing")
            array = np.asarray(weights[name])
            if array.dtype != dtype.numpy or tuple(array.shape) != lir.shape_of(shape, {}):
                raise ArgumentError(f"weight {name!r} is {array.dtype}{list(array.shape)}, expected "
                                    f"{dtype.name}{list(shape)}")
        return bound

    # -- device memory ------------------------------------------------------------------------

    def _constants(self, weights: Mapping[str, np.ndarray]) -> list[tuple]:
        """What the weight region holds: (key, host array) for each weight, packed copy and constant."""
        items = []
        for buf in self.program.buffers:
            if buf.kind == "weight":
                items.append(((buf.name, None), np.ascontiguousarray(weights[buf.name])))
            elif buf.kind == "const":
                items.append(((id(buf), None), np.ascontiguousarray(buf.value)))
        packed = {(self.program.calls[c].operands[i].buffer.name, block) for (c, i), block in self._packed.items()}
        for name, block in sorted(packed):
            items.append(((name, block), pack_rows(np.asarray(weights[name]), block)))
        return items

    def _is_resident(self, weights: Mapping[str, np.ndarray]) -> bool:
        """Whether the weight region already holds these arrays: the same objects, not equal ids.

        The uploaded arrays are held (``self._held``), so none of them can be
        freed and its id handed to a new array while it is resident. An array
        changed in place after its upload is not noticed: weights are constants.
        """
        held = self._held
        return held is not None and all(weights[name] is held[name] for name in self.program.weights)

    def _ensure(self, weights: Mapping[str, np.ndarray], call_bytes: int) -> None:
        fresh = not self._is_resident(weights)
        if fresh:
            items = self._constants(weights)
            region = sum(_align(a.nbytes) for _, a in items)
        else:
            region = self._region
        need = region + call_bytes
        if self._arena is None or self._arena.nbytes < need or fresh:
            old, old_region = self._arena, self._region
            size = max(need, (self._arena.nbytes if self._arena is not None else 0))
            self._arena = hip.DeviceArray((size,), np.uint8)
            if old is not None and not fresh:
                hip.load().nc_memcpy_d2d(self._arena.ptr, old.ptr, old_region)
            del old
        if fresh:
            self._resident.clear()
            at = 0
            for key, array in items:
                if array.nbytes:
                    hip._check(hip.load().nc_memcpy_h2d(self._arena.ptr + at, array.ctypes.data, array.nbytes),
                               "nc_memcpy_h2d")
                self._resident[key] = at
                at += _align(array.nbytes)
            self._region = region
            self._held = {name: weights[name] for name in self.program.weights}

    # -- a call -------------------------------------------------------------------------------

    def __call__(self, inputs: Mapping[str, np.ndarray], weights: Mapping[str, np.ndarray],
                 bindings: Mapping[str, int] | None = None, profile: dict | None = None) -> dict[str, np.ndarray]:
        """Run the program (runtime.py:245-301). ``profile``, if given, accumulates each
        primitive's seconds (each launch then waits for its kernel)."""
        launch, bound, addresses = self.prepare(inputs, weights, bindings)
        launch(profile=profile, inputs=inputs)
        self._wait(inputs, bound)
        lib = hip.load()
        outputs = {}
        for name, buf in self.program.outputs.items():
            out = np.empty(lir.shape_of(buf.shape, bound), buf.dtype.numpy)
            if out.nbytes:
                hip._check(lib.nc_memcpy_d2h(out.ctypes.data, addresses[buf], out.nbytes), "nc_memcpy_d2h")
            outputs[name] = out
        return outputs

    def prepare(self, inputs: Mapping[str, np.ndarray], weights: Mapping[str, np.ndarray],
                bindings: Mapping[str, int] | None = None):
        """One call's arguments checked, its buffers placed in the arena and its inputs uploaded;
        returns ``(launch, bound, addresses)``: ``launch()`` enqueues the program's kernels on the
        library stream and returns without waiting (no copies: it can be replayed, or captured
        in a graph, to time the kernels alone), ``bound`` the symbols' values, ``addresses`` each
        buffer's device address (the outputs are read from there). ``launch.calls`` holds each
        call with its launcher arguments and ``launch.symbols`` the symbol array, for a caller
        that launches calls one at a time (the autotuner).

        Lifetime: the addresses point into the arena current at this call. A later call that
        needs a larger arena, or gets new weights, moves to a new one; ``launch.arena`` keeps
        the old one allocated for as long as the launch object lives, so replaying it (or a
        graph captured from it) stays within memory it owns. Keep the launch object alive as
        long as such a graph is replayed."""
        program = self.program
        bound = self.bind(inputs, weights, bindings)
        syms = (ctypes.c_int64 * max(1, len(self.symbols)))(*[bound[s] for s in self.symbols])
        plan = plan_memory(program, self._last_use, bound)
        self.last_plan = plan
        layout = call_layout(program, bound, plan)
        hosts = {buf: np.ascontiguousarray(inputs[buf.name]) for buf in program.buffers if buf.kind == "input"}
        self._ensure(weights, layout.bytes)
        base = self._arena.ptr
        call_base = base + self._region
        addresses = {}
        for buf in program.buffers:
            if buf.kind == "weight":
                addresses[buf] = base + self._resident[(buf.name, None)]
            elif buf.kind == "const":
                addresses[buf] = base + self._resident[(id(buf), None)]
        for buf, offset in layout.offsets.items():
            addresses[buf] = call_base + offset
        lib = hip.load()
        for buf, array in hosts.items():
            if array.nbytes:
                hip._check(lib.nc_memcpy_h2d_async(addresses[buf], array.ctypes.data, array.nbytes),
                           "nc_memcpy_h2d_async")
        launches = []
        for c, call in enumerate(program.calls):
            pointers = [addresses[call.output]]
            for i, view in enumerate(call.operands):
                block = self._packed.get((c, i))
                if block is not None:
                    pointers.append(base + self._resident[(view.buffer.name, block)])
                    continue
                offset = lir.evaluate(view.offset, bound) * view.dtype.numpy.itemsize
                pointers.append(addresses[view.buffer] + offset)
            launches.append((call, (ctypes.c_void_p * len(pointers))(*pointers)))

        def launch(profile: dict | None = None, inputs=inputs) -> None:
            for call, args in launches:
                started = time.perf_counter() if profile is not None else 0.0
                status = self._launch[call.kernel](args, syms)
                if status != 0:
                    raise KernelError(f"kernel for node %{call.node} ({call.primitive}) could not be launched "
                                      f"({status}): {hip.last_error()}")
                if profile is not None:
                    self._wait(inputs, bound)
                    profile[call.primitive] = profile.get(call.primitive, 0.0) + time.perf_counter() - started

        launch.calls, launch.symbols = launches, syms
        launch.arena = self._arena          # the memory its pointers address stays allocated with it
        return launch, bound, addresses

    def _wait(self, inputs, bound) -> None:
        status = hip.load().nc_sync()
        if status == 0:
            return
        if status < 256:
            raise KernelError(f"the stream failed ({status}): {hip.last_error()}")
        kernel, code = (status >> 8) - 1, status & 0xFF
        raise self._error(kernel, code, inputs, bound)

    def _error(self, kernel: int, code: int, inputs, bound) -> KernelError:
        """A failed kernel explained from the graph node of its first call (runtime.py:303-318)."""
        for call in self.program.calls:
            if call.kernel != kernel:
                continue
            if call.gather is not None:
                rows = lir.evaluate(call.gather["rows"], bound)
                name = call.gather["ids_input"]
                if name is not None:
                    values = np.asarray(inputs[name])
                    bad = values[(values < 0) | (values >= rows)]
                    if bad.size:
                        return KernelError(f"gather index {bad.flat[0]} is outside 0..{rows - 1}")
                return KernelError(f"gather index outside 0..{rows - 1} (node %{call.node})")
            return KernelError(f"kernel for node %{call.node} ({call.primitive}) failed with {code}")
        return KernelError(f"kernel {kernel} failed with {code}")
