"""GPU autotuning: each int8 projection shape's schedule, and each generated kernel's GPU
schedule, chosen by measurement.

The reference tunes each generated C kernel over a space of CPU schedules
(autotune.py:1-53): candidates timed in alternation, medians over rounds,
weights rotated so they stream, every candidate checked bit for bit against
the unscheduled kernel, a margin before a tuned schedule replaces the
hand-written one, and a JSON cache keyed by machine and kernel. This module
keeps those rules for the GPU library:

* **The space** is the library's own schedule table, read with
  ``nc_schedule_info`` (so the tuner searches exactly what the library runs):
  GEMV launch shapes (lanes per row, waves per workgroup, 16-byte loads) and
  MFMA tiles (tile m x n, k stage, wave tile, register stages in flight,
  LDS bytes). Schedule 0, the library's own choice, is the incumbent.
* **Cost** is HIP-event time per call, on the library stream, of a captured
  graph of ``reps`` launches cycling over weight copies that together exceed
  the 256 MB Infinity Cache, so weights stream from HBM as a decode step's do.
  Candidates run in alternation, each round starting from a different one;
  the cost is the median over rounds.
* **Correctness**: each candidate runs once on random operands before it is
  timed, and its output must equal schedule 0's bit for bit; the output sits
  between two guard regions of a sentinel pattern, which must be intact after
  every candidate's run (the reference's guard regions, autotune.py:86-87,
  256-286: a schedule writing past its output fails, it is not timed).
* **Choice**: every legal candidate is measured (the space is small); the best
  then runs against the incumbent with twice the rounds and replaces it only
  if faster by more than ``margin``.
* **Dispatch**: a GPU kernel's schedule is chosen per call, so the tuner picks
  per token count M (decode and each prefill length) rather than one schedule
  scored over a mix of workloads (the reference's DECODE/PREFILL weights,
  autotune.py:65-69, exist because its C is compiled once for all seq).
* **The cache** is JSON keyed by machine (arch, HIP runtime and driver
  versions, CU count) and by problem (op, M, N, K, the space, and the
  library's digest of its kernel sources and flags, so a rebuilt kernel is
  measured afresh).

Generated kernels (codegen_hip) are tuned the same way over the code
generator's schedule space (gpu_schedule.space: workgroup size, LDS staging,
workgroup items with one lead wave and hoisted chain operands, accumulators
across lanes, weight packing, vector width, unroll), per kernel of a
program, on weighted workloads of symbol values as the reference does
(``Autotuner.schedule_program``; see ``tune_program``).
"""

from __future__ import annotations

import hashlib
import json
import os
import statistics
import sys
import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from nanocompile_amd import hip, kernels
from nanocompile_amd.hip import DeviceArray, Event, Graph

OPS = ("matmul_i8_token", "matmul_i8_token_swiglu")
STREAM_BYTES = 512 * 2**20      # weight bytes one sample cycles through: past the 256 MB Infinity Cache
MAX_COPIES = 64
CACHE_VERSION = 1
GUARD = 4096                    # float32 words of sentinel before and after a candidate's output
SENTINEL = 0x7FC0DEAD           # a quiet NaN's bits: no projection writes it


class TuningError(RuntimeError):
    """A candidate failed its bit-for-bit check or its guard regions, or could not be measured."""


def guarded(words: int) -> np.ndarray:
    """An output of ``words`` float32 words between two guard regions, as host bits to upload."""
    return np.full(GUARD + words + GUARD, SENTINEL, np.uint32)


def guards_broken(bits: np.ndarray) -> list[int]:
    """Word offsets, relative to the output's first word, of guard words that are not the sentinel."""
    bits = np.asarray(bits, np.uint32)
    head, tail = bits[:GUARD], bits[len(bits) - GUARD:]
    return ([int(i) - GUARD for i in np.flatnonzero(head != SENTINEL)] +
            [int(i) + len(bits) - 2 * GUARD for i in np.flatnonzero(tail != SENTINEL)])


# -- the space ---------------------------------------------------------------------------


def legal_space(op: str, m: int, n: int, k: int) -> list[dict]:
    """Schedule 0 (the library's choice) first, then every schedule that applies to this problem."""
    if op not in OPS:
        raise ValueError(f"no tuning space for {op!r}")
    out = [{"schedule": 0, "kernel": "default"}]
    gemv = list(kernels.GEMV_SCHEDULES) if op == "matmul_i8_token" else [7]
    for s in gemv:
        out.append(hip.schedule_info(s))
    if k % 16 == 0 and (op == "matmul_i8_token" or k <= 8192):
        for s in kernels.GEMM_SCHEDULES:
            out.append(hip.schedule_info(s))
    return out


# -- the problem on the device -------------------------------------------------------------


class Problem:
    """Device operands for one projection shape, with its weights in rotating copies."""

    def __init__(self, op: str, m: int, n: int, k: int, seed: int = 0,
                 stream_bytes: int = STREAM_BYTES) -> None:
        self.op, self.m, self.n, self.k = op, m, n, k
        self.shape = (m, n, k)
        rng = np.random.default_rng(seed)
        per_copy = n * k * (2 if op == "matmul_i8_token_swiglu" else 1)
        self.copies = int(min(MAX_COPIES, max(2, -(-stream_bytes // max(per_copy, 1)))))
        self.xq = DeviceArray.from_host(rng.integers(-127, 128, (m, k)).astype(np.int8))
        self.xs = DeviceArray.from_host((rng.random(m) * 0.05 + 1e-3).astype(np.float32))
        matrices = 2 if op == "matmul_i8_token_swiglu" else 1
        host = [rng.integers(-127, 128, (n, k)).astype(np.int8) for _ in range(matrices)]
        self.q = [[DeviceArray.from_host(w) for w in host] for _ in range(self.copies)]
        self.scales = [DeviceArray.from_host((rng.random(n) * 1e-3).astype(np.float32)) for _ in range(matrices)]
        self.bias = DeviceArray.from_host(rng.standard_normal(n).astype(np.float32))
        self.guarded = DeviceArray.from_host(guarded(m * n))
        self.y = self.guarded.view((m, n), np.float32, offset_bytes=GUARD * 4)

    def launch(self, schedule: int, copy: int = 0) -> None:
        q = self.q[copy % self.copies]
        if self.op == "matmul_i8_token":
            hip.call("nc_matmul_i8_token", [self.y, self.xq, self.xs, q[0], self.scales[0], self.bias, None],
                     [self.m, self.n, self.k, schedule])
        else:
            hip.call("nc_matmul_i8_token_swiglu",
                     [self.y, self.xq, self.xs, q[0], self.scales[0], q[1], self.scales[1]],
                     [self.m, self.n, self.k, schedule])

    def space(self) -> list[dict]:
        return legal_space(self.op, self.m, self.n, self.k)

    def output(self, schedule: int) -> np.ndarray:
        """The schedule's output bits; TuningError if it wrote into a guard region."""
        self.guarded.upload(guarded(self.m * self.n))
        self.launch(schedule, 0)
        return checked_output(self, schedule, self.guarded, self.m * self.n)


def checked_output(problem, schedule: int, region: DeviceArray, words: int) -> np.ndarray:
    """After a launch into ``region`` (GUARD words, the output, GUARD words): the output's bits,
    or TuningError if a guard word changed."""
    hip.sync()
    bits = region.numpy()
    broken = guards_broken(bits)
    if broken:
        raise TuningError(f"{problem.op} schedule {schedule} on {problem.shape} wrote outside its output, "
                          f"at word offsets {broken[:4]}")
    return bits[GUARD:GUARD + words].copy()


class DecodeProblem:
    """One decode projection (nc_decode_projection) of ``kind`` over N rows of width K: the step's
    activation row, its prologue and epilogue operands, and the weights in rotating copies so they
    stream from HBM as a decode step's do. Kinds: 0 rms_norm + bias (q, k, v), 1 quantize +
    residual (o, down), 2 rms_norm + SwiGLU pair (gate, up)."""

    op = "decode_projection"

    def __init__(self, kind: int, n: int, k: int, seed: int = 0, stream_bytes: int = STREAM_BYTES) -> None:
        self.kind, self.n, self.k = kind, n, k
        self.shape = (kind, n, k)
        rng = np.random.default_rng(seed)
        matrices = 2 if kind == 2 else 1
        self.copies = int(min(MAX_COPIES, max(2, -(-stream_bytes // max(n * k * matrices, 1)))))
        self.x = DeviceArray.from_host(rng.standard_normal(k).astype(np.float32))
        self.gamma = DeviceArray.from_host((1 + 0.1 * rng.standard_normal(k)).astype(np.float32))
        host = [rng.integers(-127, 128, (n, k)).astype(np.int8) for _ in range(matrices)]
        self.q = [[DeviceArray.from_host(w) for w in host] for _ in range(self.copies)]
        self.scales = [DeviceArray.from_host((rng.random(n) * 1e-3).astype(np.float32)) for _ in range(matrices)]
        self.bias = DeviceArray.from_host(rng.standard_normal(n).astype(np.float32))
        self.residual = rng.standard_normal(n).astype(np.float32)
        self.guarded = DeviceArray.from_host(guarded(n))
        self.y = self.guarded.view((n,), np.float32, offset_bytes=GUARD * 4)

    def space(self) -> list[dict]:
        out = [{"schedule": 0, "kernel": "default"}]
        for s in range(1, 8):
            shape = hip.decode_schedule_info(self.k, self.kind, s)
            if shape is not None:
                out.append({"schedule": s, "kernel": "gemv_decode", **shape})
        return out

    def launch(self, schedule: int, copy: int = 0) -> None:
        from nanocompile_amd.kernels import float_bits
        q = self.q[copy % self.copies]
        gamma = None if self.kind == 1 else self.gamma
        bias = self.bias if self.kind == 0 else None
        q2, s2 = (q[1], self.scales[1]) if self.kind == 2 else (None, None)
        hip.call("nc_decode_projection", [self.y, self.x, gamma, q[0], self.scales[0], bias, q2, s2],
                 [self.n, self.k, self.kind, float_bits(1e-6), schedule])

    def output(self, schedule: int) -> np.ndarray:
        bits = guarded(self.n)
        if self.kind == 1:                       # the output holds the residual the projection adds to
            bits[GUARD:GUARD + self.n] = self.residual.view(np.uint32)
        self.guarded.upload(bits)
        self.launch(schedule, 0)
        return checked_output(self, schedule, self.guarded, self.n)


class AttentionProblem:
    """A prompt's attention (nc_attention) over M rows at past 0 with heads / kv heads of width D:
    rotated q, k and v rows, the cache holding the prompt's keys and values, the chunk workspace."""

    op = "attention_prefill"

    def __init__(self, m: int, heads: int, kv: int, d: int, seed: int = 0) -> None:
        from nanocompile_amd.kernels import attention_workspace_bytes
        self.m, self.heads, self.kv, self.d = m, heads, kv, d
        self.shape = (m, heads, kv, d)
        rng = np.random.default_rng(seed)
        self.qkv = DeviceArray.from_host(rng.standard_normal((m, (heads + 2 * kv) * d)).astype(np.float32))
        self.kc = DeviceArray.from_host(rng.standard_normal((kv, m, d)).astype(np.float32))
        self.vc = DeviceArray.from_host(rng.standard_normal((kv, m, d)).astype(np.float32))
        self.work_bytes = attention_workspace_bytes(heads, d, m, m)
        self.work = DeviceArray((self.work_bytes // 4,), np.float32)
        self.guarded = DeviceArray.from_host(guarded(m * heads * d))
        self.ctx = self.guarded.view((m, heads * d), np.float32, offset_bytes=GUARD * 4)

    def space(self) -> list[dict]:
        out = [{"schedule": 0, "kernel": "default"}]
        for s in range(1, 8):
            rows = hip.attention_schedule_info(s)
            if rows is not None:
                out.append({"schedule": s, "kernel": "attention_rows_chunks", "rows": rows})
        return out

    def launch(self, schedule: int, copy: int = 0) -> None:
        from nanocompile_amd.kernels import float_bits
        hip.call("nc_attention", [self.ctx, self.qkv, self.kc, self.vc, None, self.work],
                 [self.m, self.heads, self.kv, self.d, 0, self.m, float_bits(self.d ** -0.5), self.work_bytes,
                  schedule])

    def output(self, schedule: int) -> np.ndarray:
        self.guarded.upload(guarded(self.m * self.heads * self.d))
        self.launch(schedule, 0)
        return checked_output(self, schedule, self.guarded, self.m * self.heads * self.d)


class RopeProblem:
    """A prompt's qkv projection with RoPE and the KV-cache append in its epilogue
    (nc_matmul_i8_token_rope) over M rows at past 0, W = (heads + 2 kv) D rows of width K: the
    int8 activations, the weights in rotating copies, the cache and RoPE's table. Its space is
    the MFMA tiles one head wide (the epilogue rotates a tile as a head)."""

    op = "qkv_rope"

    def __init__(self, m: int, w: int, k: int, heads: int, kv: int, d: int, seed: int = 0,
                 stream_bytes: int = STREAM_BYTES) -> None:
        from nanocompile_amd.models.qwen2 import inverse_frequencies
        self.m, self.w, self.k, self.heads, self.kv, self.d = m, w, k, heads, kv, d
        self.shape = (m, w, k, heads, kv, d)
        rng = np.random.default_rng(seed)
        self.copies = int(min(MAX_COPIES, max(2, -(-stream_bytes // max(w * k, 1)))))
        self.xq = DeviceArray.from_host(rng.integers(-127, 128, (m, k)).astype(np.int8))
        self.xs = DeviceArray.from_host((rng.random(m) * 0.05 + 1e-3).astype(np.float32))
        host = rng.integers(-127, 128, (w, k)).astype(np.int8)
        self.q = [DeviceArray.from_host(host) for _ in range(self.copies)]
        self.scales = DeviceArray.from_host((rng.random(w) * 1e-3).astype(np.float32))
        self.bias = DeviceArray.from_host(rng.standard_normal(w).astype(np.float32))
        self.kc, self.vc = DeviceArray((kv, m, d), np.float32), DeviceArray((kv, m, d), np.float32)
        self.table = DeviceArray((2, m, d // 2), np.float32)
        hip.call("nc_rope_table", [self.table, DeviceArray.from_host(inverse_frequencies(d, 1e6))], [m, d])
        self.guarded = DeviceArray.from_host(guarded(m * w))
        self.y = self.guarded.view((m, w), np.float32, offset_bytes=GUARD * 4)

    def space(self) -> list[dict]:
        out = [{"schedule": 0, "kernel": "default"}]
        for s in kernels.GEMM_SCHEDULES:
            shape = hip.schedule_info(s)
            if shape["tile_n"] == self.d and self.k % 16 == 0:
                out.append(shape)
        return out

    def launch(self, schedule: int, copy: int = 0) -> None:
        hip.call("nc_matmul_i8_token_rope",
                 [self.y, self.xq, self.xs, self.q[copy % self.copies], self.scales, self.bias, self.kc, self.vc,
                  self.table, None],
                 [self.m, self.w, self.k, self.heads, self.kv, self.d, 0, self.m, schedule])

    def output(self, schedule: int) -> np.ndarray:
        """The rotated qkv rows and both caches' bits; TuningError if qkv's guards were written."""
        self.guarded.upload(guarded(self.m * self.w))
        self.launch(schedule, 0)
        bits = checked_output(self, schedule, self.guarded, self.m * self.w)
        return np.concatenate([bits, self.kc.numpy().view(np.uint32).ravel(), self.vc.numpy().view(np.uint32).ravel()])


def measure(problem: Problem, schedules: list[int], rounds: int, reps: int, progress=None) -> list[float]:
    """Median seconds per call of each schedule, the candidates alternating round by round
    (``progress()``, when given, after each sample)."""
    graphs = {}
    for s in schedules:
        graphs[s] = Graph.capture(lambda s=s: [problem.launch(s, i) for i in range(reps)])
        graphs[s].launch()                      # warm: code objects loaded, caches in steady state
    hip.sync()
    start, stop = Event(), Event()
    samples: dict[int, list[float]] = {s: [] for s in schedules}
    for r in range(rounds):
        order = schedules[r % len(schedules):] + schedules[:r % len(schedules)]
        for s in order:
            start.record()
            graphs[s].launch()
            stop.record()
            hip.sync()
            samples[s].append(start.elapsed_ms(stop) * 1e-3 / reps)
            if progress is not None:
                progress()
    return [statistics.median(samples[s]) for s in schedules]


# -- decisions, their log, and the cache ----------------------------------------------------------


@dataclass(frozen=True)
class Evaluation:
    """One timing pass of ``choose``: the candidates it ran and their seconds per call."""

    stage: str
    schedules: list[int]
    costs: list[float]


@dataclass(frozen=True)
class TuneRecord:
    """The answer to one tuning question, measured now or read back from the cache.

    ``winner`` is a schedule number (a library problem) or a candidate index
    whose point of the schedule space is ``config`` (a generated kernel).
    ``costs`` holds (incumbent, winner) in seconds per call, or per token for a
    generated kernel's weighted workloads; ``None`` where they are unknown.
    ``evaluations`` is what ``choose`` timed, empty for a cached answer.
    """

    key: str
    op: str
    shape: tuple
    space_size: int
    winner: int = 0
    costs: tuple = (None, None)
    cached: bool = False
    config: dict | None = None
    evaluations: tuple = ()
    seconds: float = 0.0

    @property
    def default_cost(self) -> float | None:
        return self.costs[0]

    @property
    def winner_cost(self) -> float | None:
        return self.costs[1]

    @property
    def speedup(self) -> float | None:
        before, after = self.costs
        return before / after if before and after else None


def choose(space: list[int], cost, margin: float) -> tuple[int, list[Evaluation], float, float]:
    """Measure every candidate, then the best against the incumbent (space[0]) with more rounds.

    ``cost(stage, schedules)`` returns seconds per call. The best replaces the
    incumbent only if it is faster by more than ``margin``; returns (winner,
    evaluations, incumbent's cost, winner's cost).
    """
    incumbent = space[0]
    log = []
    costs = cost("sample", list(space))
    log.append(Evaluation("sample", list(space), costs))
    best = space[int(np.argmin(costs))]
    if best == incumbent:
        return incumbent, log, costs[0], costs[0]
    confirm = cost("confirm", [incumbent, best])
    log.append(Evaluation("confirm", [incumbent, best], confirm))
    if confirm[1] < confirm[0] * (1.0 - margin):
        return best, log, confirm[0], confirm[1]
    return incumbent, log, confirm[0], confirm[0]


# how many of the tuner's rounds each stage of ``choose`` runs: the confirmation decides, so it
# gets more samples than the first pass over every candidate
ROUNDS_FACTOR = {"sample": 1, "confirm": 2}


def machine_key() -> str:
    """Arch, HIP runtime and driver, CU count: a schedule tuned on one need not suit another."""
    info = hip.device_info()
    runtime, driver = hip.runtime_version()
    material = f"{info['arch']}|{runtime}|{driver}|{info['compute_units']}"
    return hashlib.sha256(material.encode()).hexdigest()[:16]


class TuningCache:
    """Tuning answers on disk, as an append-only log of JSON lines.

    Each ``put`` appends one line, ``{"v": CACHE_VERSION, "machine": ..., "key":
    ..., "entry": {...}}``, in a single write to a file opened for appending, so
    tuners in several processes never overwrite each other's answers and a crash
    loses at most the line being written. ``get`` scans the log and returns the
    newest entry for (machine, key). Lines of another version, torn lines and
    anything that is not such an object are skipped, so a damaged or foreign
    file reads as fewer answers, never as an error.
    """

    def __init__(self, path: Path | str | None = None) -> None:
        if path is None:
            path = os.environ.get("NANOCOMPILE_AMD_TUNING") or (
                Path.home() / ".cache" / "nanocompile_amd" / "tuning.jsonl")
        self.path = Path(path)

    def _answers(self):
        try:
            raw = self.path.read_bytes()
        except (FileNotFoundError, IsADirectoryError):
            return
        for line in raw.split(b"\n"):
            try:
                item = json.loads(line)
            except (ValueError, RecursionError):
                continue
            if isinstance(item, dict) and item.get("v") == CACHE_VERSION and isinstance(item.get("entry"), dict):
                yield item

    def get(self, machine: str, key: str) -> dict | None:
        newest = None
        for item in self._answers():
            if item.get("machine") == machine and item.get("key") == key:
                newest = item["entry"]
        return newest

    def put(self, machine: str, key: str, entry: dict) -> None:
        line = json.dumps({"v": CACHE_VERSION, "machine": machine, "key": key, "entry": entry}, sort_keys=True)
        self.path.parent.mkdir(parents=True, exist_ok=True)
        fd = os.open(self.path, os.O_RDWR | os.O_CREAT | os.O_APPEND, 0o644)
        try:
            size = os.fstat(fd).st_size
            # a torn last line (no newline) is closed first, so this answer starts a line of its own
            torn = size > 0 and os.pread(fd, 1, size - 1) != b"\n"
            os.write(fd, (b"\n" if torn else b"") + line.encode() + b"\n")
        finally:
            os.close(fd)


# -- generated kernels: the code generator's schedule space ------------------------------------

# A workload: (name, symbol values, weight); the weight turns seconds per call into seconds per
# token, so a decode step and a prefill add up (the reference's DECODE and PREFILL, autotune.py:65-69).
DECODE = ("decode", {"seq": 1, "past": 64}, 1.0)
PREFILL = ("prefill", {"seq": 32, "past": 0}, 1.0 / 32)
WORKLOADS = (DECODE, PREFILL)
SENTINEL_BYTE = 0xA5             # a candidate's output is filled with it before the candidate runs
WHOLE_ARENA = 64 * 2**20         # arenas up to this size are compared whole after each candidate
GUARD_BYTES = 1 * 2**20          # else the output and this much either side of it


@dataclass
class Candidate:
    """One point of a generated kernel's schedule space (gpu_schedule.space): its configuration,
    the scheduled kernel and launch, and the kernel's generated text."""

    config: dict
    kernel: object
    launch: object
    source: str


def kernel_candidates(kernel, calls) -> list[Candidate]:
    """The points of ``kernel``'s space that apply, the default schedule first, one per distinct
    generated kernel (the reference's legal_space, autotune.py:571-590). A candidate runs on the
    default's arguments, so points that would read packed an operand the default reads row-major
    are left out (the packed copy would not be there); the other way round is allowed, the
    row-major copy of every weight being resident."""
    from nanocompile_amd import codegen_hip, gpu_schedule
    first = gpu_schedule.default_config(kernel, calls)
    out, seen, base = [], set(), None
    for config in [first] + [c for c in gpu_schedule.space(kernel) if c != first]:
        try:
            scheduled, launch = gpu_schedule.apply(kernel, calls, config)
        except gpu_schedule.ScheduleError:
            continue
        packs = [p.packed for p in scheduled.params]
        if base is None:
            base = packs
        elif any(p is not None and p != b for p, b in zip(packs, base)):
            continue
        source = codegen_hip.render_kernel(scheduled, launch, 0)
        if source in seen:
            continue
        seen.add(source)
        out.append(Candidate(config, scheduled, launch, source))
    return out


class CandidateLibrary:
    """Every candidate of every kernel of a program, generated into one library.

    ``entry[i][c]`` is the launcher (``nc_k<entry>``) of kernel ``i``'s
    candidate ``c``; candidate 0 is the default schedule. The candidates are
    measured in this library and the chosen ones run from it, so a tuned
    program needs no second compile.
    """

    def __init__(self, program) -> None:
        from nanocompile_amd import codegen_hip, lir
        program = lir.adapt(program)
        calls_of: dict[int, list] = {}
        for call in program.calls:
            calls_of.setdefault(call.kernel, []).append(call)
        self.program = program
        self.calls_of = calls_of
        self.candidates = [kernel_candidates(k, calls_of.get(i, [])) for i, k in enumerate(program.kernels)]
        for i, cands in enumerate(self.candidates):
            # the tuner runs a candidate on the default's arguments, an operand the default reads
            # packed pointed at its row-major copy where the candidate reads it so
            default = [p.packed for p in cands[0].kernel.params]
            for c in cands[1:]:
                if any(p.packed is not None and p.packed != d for p, d in zip(c.kernel.params, default)):
                    raise TuningError(f"kernel {i}: a candidate packs an operand the default does not")
        scheduled, owners, self.entry = [], [], []
        for i, cands in enumerate(self.candidates):
            self.entry.append([])
            for c in cands:
                self.entry[i].append(len(scheduled))
                scheduled.append((c.kernel, c.launch))
                owners.append(i)
        self.source = codegen_hip.render_library(scheduled, owners)

    def build(self):
        """(path, was it cached) of the built library (codegen_hip.build_library)."""
        from nanocompile_amd import codegen_hip
        return codegen_hip.build_library(self.source)

    def choice(self, chosen) -> tuple:
        """``(scheduled, source, launcher names)`` with kernel ``i`` at candidate ``chosen[i]``."""
        from nanocompile_amd import codegen_hip
        scheduled = [(self.candidates[i][c].kernel, self.candidates[i][c].launch) for i, c in enumerate(chosen)]
        names = [codegen_hip.kernel_name(self.entry[i][c]) for i, c in enumerate(chosen)]
        return scheduled, self.source, names


class Chosen:
    """A schedule for CompiledProgram: kernel ``i`` at candidate ``chosen[i]`` of ``library``."""

    def __init__(self, library: CandidateLibrary, chosen) -> None:
        self.library, self.chosen = library, list(chosen)

    def library_for(self, program) -> tuple:
        return self.library.choice(self.chosen)


def random_arguments(program, bindings, rng) -> tuple[dict, dict, dict]:
    """Inputs and weights of a program's interface at ``bindings``: floats normal, int8 and bool
    uniform, wider integers zero (they index: ids, positions), so every gather is in range."""
    from nanocompile_amd import lir

    def draw(shape, dtype):
        if dtype.name == "f32":
            return rng.standard_normal(shape, dtype=np.float32)
        if dtype.name == "i8":
            return rng.integers(-127, 128, shape, dtype=np.int8)
        if dtype.name == "bool":
            return rng.integers(0, 2, shape).astype(dtype.numpy)
        return np.zeros(shape, dtype.numpy)

    bound = {name: int(v) for name, v in bindings.items() if name in program.symbols}
    missing = [name for name in program.symbols if name not in bound]
    if missing:
        raise TuningError(f"the workload {dict(bindings)} gives no value to {missing}")
    inputs = {name: draw(lir.shape_of(shape, bound), dtype) for name, dtype, shape in program.inputs}
    weights = {name: draw(lir.shape_of(shape, {}), dtype) for name, (dtype, shape) in program.weights.items()}
    return inputs, weights, bound


class ProgramWorkload:
    """A program on the device at one workload's symbols, for timing its kernels' candidates:
    every call's arguments placed in one arena (the default schedules' outputs in place)."""

    def __init__(self, library: CandidateLibrary, bindings, seed: int) -> None:
        from nanocompile_amd import compiled
        self.library = library
        program = library.program
        self.compiled = compiled.CompiledProgram(program, Chosen(library, [0] * len(program.kernels)))
        lib = self.compiled._library
        self.launchers = [[compiled.KERNEL_TYPE((f"nc_k{n}", lib)) for n in entries] for entries in library.entry]
        inputs, weights, bound = random_arguments(program, bindings, np.random.default_rng(seed))
        self.launch, self.bound, self.addresses = self.compiled.prepare(inputs, weights, bound)
        self.calls = self.launch.calls
        self.symbols = self.launch.symbols
        self.inputs = inputs
        self._args: dict = {}

    def _layout_args(self, call, args, candidate):
        """The call's launcher arguments for a candidate that reads a weight row-major where the
        default reads it packed (the row-major copy is always resident): the default's, with those
        operands pointed at the row-major copy. Packing where the default does not is refused."""
        import ctypes

        from nanocompile_amd import lir
        params = candidate.kernel.params
        default = self.library.candidates[call.kernel][0].kernel.params
        if all(p.packed == q.packed for p, q in zip(params, default)):
            return args
        key = (id(args), tuple(p.packed for p in params))
        if key not in self._args:
            pointers = [args[i] for i in range(len(params))]
            for i, view in enumerate(call.operands):
                ours, theirs = params[i + 1].packed, default[i + 1].packed
                if ours == theirs:
                    continue
                if ours is not None:
                    raise TuningError(f"kernel {call.kernel}: a candidate packs an operand the default does not")
                offset = lir.evaluate(view.offset, self.bound) * view.dtype.numpy.itemsize
                pointers[i + 1] = self.addresses[view.buffer] + offset
            self._args[key] = (ctypes.c_void_p * len(pointers))(*pointers)
        return self._args[key]

    def _run(self, kernel: int, candidate: int, args, call=None) -> None:
        if call is not None and candidate:
            args = self._layout_args(call, args, self.library.candidates[kernel][candidate])
        status = self.launchers[kernel][candidate](args, self.symbols)
        if status != 0:
            raise TuningError(f"kernel {kernel} candidate {candidate} could not be launched ({status}): "
                              f"{hip.last_error()}")

    def gate(self, kernels) -> None:
        """Run the program's calls in order on the default schedules; at the first call of each
        kernel in ``kernels``, run every other candidate on the same arguments, its output filled
        with a sentinel first: the arena must then hold exactly what the default left (its
        output bit for bit, every other byte untouched). The whole arena is compared up to
        WHOLE_ARENA bytes; above that, the output and GUARD_BYTES either side of it."""
        from nanocompile_amd.compiled import _nbytes
        pending = set(kernels)
        arena = self.compiled._arena
        base = arena.ptr
        lib = hip.load()
        for call, args in self.calls:
            self._run(call.kernel, 0, args)
            hip.sync()
            if call.kernel not in pending:
                continue
            pending.discard(call.kernel)
            at, n = self.addresses[call.output] - base, _nbytes(call.output, self.bound)
            if arena.nbytes <= WHOLE_ARENA:
                lo, hi = 0, arena.nbytes
            else:
                lo, hi = max(0, at - GUARD_BYTES), min(arena.nbytes, at + n + GUARD_BYTES)
            window = arena.view((hi - lo,), np.uint8, offset_bytes=lo)
            before = window.numpy().copy()
            fill = np.full(max(n, 1), SENTINEL_BYTE, np.uint8)
            for c in range(1, len(self.launchers[call.kernel])):
                if n:
                    hip._check(lib.nc_memcpy_h2d(base + at, fill.ctypes.data, n), "nc_memcpy_h2d")
                self._run(call.kernel, c, args, call)
                hip.sync()
                after = window.numpy()
                if not np.array_equal(after, before):
                    diff = np.flatnonzero(after != before)
                    first = int(diff[0]) + lo
                    where = "its output" if at <= first < at + n else "outside its output"
                    config = self.library.candidates[call.kernel][c].config
                    raise TuningError(f"kernel {call.kernel} ({call.primitive}) candidate {c} {config} differs "
                                      f"from the default schedule at byte {first - at} of {n} ({where})")

    def timer(self, kernel: int):
        """An object ``measure`` times: ``launch(candidate, copy)`` runs kernel ``kernel``'s calls."""
        calls = [(call, a) for call, a in self.calls if call.kernel == kernel]
        workload = self

        class Calls:
            def launch(self, candidate: int, copy: int = 0) -> None:
                for call, a in calls:
                    workload._run(kernel, candidate, a, call)

        return Calls()


def program_kernel_key(library: CandidateLibrary, kernel: int, workloads) -> str:
    """A generated kernel's cache key: its candidates' text, what its calls read, the workloads
    and the compiler (the reference's kernel_key, autotune.py:548-560)."""
    from nanocompile_amd import codegen_hip
    calls = library.calls_of.get(kernel, [])
    operands = [[v.buffer.kind, v.buffer.dtype.name, [str(d) for d in v.buffer.shape], str(v.offset)]
                for v in calls[0].operands] if calls else []
    material = json.dumps({
        "candidates": [c.source for c in library.candidates[kernel]],
        "operands": operands,
        "symbols": list(library.program.symbols),
        "workloads": [[n, sorted(b.items()), w] for n, b, w in workloads],
        "compiler": codegen_hip.compiler_identity(codegen_hip.hipcc()),
        "flags": list(codegen_hip.HIPCC_FLAGS),
    }, sort_keys=True)
    return hashlib.sha256(material.encode()).hexdigest()[:20]


# -- the tuner --------------------------------------------------------------------------------


class Autotuner:
    """Finds, by timing on the GPU in use, the fastest schedule of each problem it is asked
    about: a projection (op, M, N, K), a prompt's attention, a generated program's kernels.

    Winners persist through ``cache``: a TuningCache; a file path; True for the file that
    NANOCOMPILE_AMD_TUNING names, else one under the user's cache directory; or None, which
    keeps nothing across processes, so each new tuner times each problem again. ``records``
    lists every tuning this tuner ran or read back.
    """

    def __init__(self, rounds: int = 7, reps: int = 32, margin: float = 0.03, seed: int = 0,
                 cache: TuningCache | Path | str | bool | None = True, verbose: bool = False,
                 stream_bytes: int = STREAM_BYTES, workloads=None) -> None:
        self.rounds, self.reps, self.margin, self.seed = rounds, reps, margin, seed
        self.workloads = tuple(WORKLOADS if workloads is None else workloads)
        if cache is True:
            cache = TuningCache()
        elif cache not in (None, False) and not isinstance(cache, TuningCache):
            cache = TuningCache(cache)
        self.cache: TuningCache | None = cache or None
        self.verbose = verbose
        self.stream_bytes = stream_bytes
        self.records: list[TuneRecord] = []
        self._chosen: dict[tuple, int] = {}

    @staticmethod
    def problem_key(op: str, m: int, n: int, k: int, space: list[dict], extra: tuple = ()) -> str:
        material = json.dumps({"op": op, "m": m, "n": n, "k": k, "space": space, "extra": list(extra),
                               "library": hip.library_digest()}, sort_keys=True)
        return hashlib.sha256(material.encode()).hexdigest()[:20]

    def schedule(self, op: str, m: int, n: int, k: int) -> int:
        """The schedule to launch ``op`` with on an [m, k] x [n, k]^T problem (tuned once, then remembered)."""
        at = (op, m, n, k)
        if at not in self._chosen:
            self._chosen[at] = self.tune(op, m, n, k).winner
        return self._chosen[at]

    def tune(self, op: str, m: int, n: int, k: int) -> TuneRecord:
        """Tune a projection (``matmul_i8_token`` or ``matmul_i8_token_swiglu``) on an [m, k] x [n, k]^T problem."""
        if op not in OPS:
            raise ValueError(f"no tuning space for {op!r}")
        return self.tune_problem(lambda: Problem(op, m, n, k, self.seed, self.stream_bytes), op, (m, n, k),
                                 legal_space(op, m, n, k))

    def decode_schedule(self, kind: int, n: int, k: int) -> int:
        """The schedule of a decode projection (nc_decode_projection's kind, N rows, width K)."""
        at = ("decode_projection", kind, n, k)
        if at not in self._chosen:
            self._chosen[at] = self.tune_problem(
                lambda: DecodeProblem(kind, n, k, self.seed, self.stream_bytes), "decode_projection", (kind, n, k),
                None).winner
        return self._chosen[at]

    def attention_schedule(self, m: int, heads: int, kv: int, d: int) -> int:
        """The schedule of a prompt's attention (nc_attention) over m rows at past 0."""
        at = ("attention_prefill", m, heads, kv, d)
        if at not in self._chosen:
            self._chosen[at] = self.tune_problem(lambda: AttentionProblem(m, heads, kv, d, self.seed),
                                                 "attention_prefill", (m, heads, kv, d), None).winner
        return self._chosen[at]

    def rope_schedule(self, m: int, w: int, k: int, heads: int, kv: int, d: int) -> int:
        """The schedule of a prompt's qkv projection with RoPE in its epilogue (nc_matmul_i8_token_rope)."""
        at = ("qkv_rope", m, w, k, heads, kv, d)
        if at not in self._chosen:
            self._chosen[at] = self.tune_problem(
                lambda: RopeProblem(m, w, k, heads, kv, d, self.seed, self.stream_bytes), "qkv_rope",
                (m, w, k, heads, kv, d), None).winner
        return self._chosen[at]

    # -- generated programs ------------------------------------------------------------------

    def schedule_program(self, program) -> list:
        """[(kernel, Launch)] of ``program`` with each kernel at its measured best schedule."""
        library, chosen = self.tune_program(program)
        return library.choice(chosen)[0]

    def library_for(self, program) -> tuple:
        """For CompiledProgram: the tuned kernels, run from the library they were measured in."""
        library, chosen = self.tune_program(program)
        return library.choice(chosen)

    def tune_program(self, program) -> tuple[CandidateLibrary, list[int]]:
        """Choose each kernel's schedule from its space (gpu_schedule.space) by measurement.

        All candidates of all kernels are generated into one library. For each
        workload (symbol values, weighted per token) the program runs on random
        inputs; at each kernel's first call every candidate is checked against
        the default schedule on the same arguments (``ProgramWorkload.gate``),
        then the candidates of each kernel are timed on all of its calls, in
        alternation over rounds, and ``choose`` keeps the default unless the
        best beats it by more than ``margin``. A cached kernel is not measured.
        """
        library = CandidateLibrary(program)
        chosen = [0] * len(library.candidates)
        keys = [program_kernel_key(library, i, self.workloads) for i in range(len(chosen))]
        machine = machine_key()
        todo = []
        for i, cands in enumerate(library.candidates):
            if len(cands) <= 1 or not library.calls_of.get(i):
                continue                               # nothing to choose, or never called
            answer = self._recall(machine, keys[i])
            stored = answer.get("config") if answer is not None else None
            match = next((c for c, cand in enumerate(cands) if isinstance(stored, dict)
                          and sorted(cand.config.items()) == sorted(stored.items())), None)
            if match is None:
                todo.append(i)                         # never tuned here, or its point left the space
                continue
            chosen[i] = match
            self._log(TuneRecord(keys[i], library.program.kernels[i].primitive, (i,), len(cands), match,
                                 (answer.get("default_cost"), answer.get("winner_cost")), cached=True,
                                 config=stored))
        if not todo:
            return library, chosen
        clock = time.perf_counter()
        workloads = [(ProgramWorkload(library, bindings, self.seed + w), weight)
                     for w, (_, bindings, weight) in enumerate(self.workloads)]
        for workload, _ in workloads:
            workload.gate(todo)
        for i in todo:
            began = time.perf_counter()
            cands = library.candidates[i]
            progress = self._progress(i, len(cands)) if self.verbose else None
            cost = self._cost([(workload.timer(i), weight) for workload, weight in workloads], progress)
            winner, trail, before, after = choose(list(range(len(cands))), cost, self.margin)
            chosen[i] = winner
            record = self._log(TuneRecord(keys[i], library.program.kernels[i].primitive, (i,), len(cands), winner,
                                          (before, after), config=cands[winner].config, evaluations=tuple(trail),
                                          seconds=time.perf_counter() - began))
            self._remember(machine, keys[i], {"config": record.config, "default_cost": before,
                                              "winner_cost": after, "op": record.op})
            if self.verbose:
                print(f"tuned kernel {i} ({record.op}): {len(cands)} schedules, "
                      f"{cands[winner].launch.describe()} at {after * 1e6:.2f} us per token "
                      f"({record.speedup:.2f}x the default)", file=sys.stderr, flush=True)
        if self.verbose:
            print(f"tuned {len(todo)} generated kernels in {time.perf_counter() - clock:.1f} s", file=sys.stderr,
                  flush=True)
        return library, chosen

    @staticmethod
    def _progress(kernel: int, total: int, seconds: float = 20.0):
        """A ``measure`` progress callback that prints a line when a sample completes at least
        ``seconds`` after the last line (a kernel whose candidates run for milliseconds each
        takes minutes to tune; one that tunes in seconds prints nothing)."""
        done, last = [0], [time.perf_counter()]

        def sampled() -> None:
            done[0] += 1
            now = time.perf_counter()
            if now - last[0] >= seconds:
                last[0] = now
                print(f"tuning kernel {kernel}: {done[0]} samples taken ({total} schedules)", file=sys.stderr,
                      flush=True)
        return sampled

    # -- shared steps ----------------------------------------------------------------------------

    def _log(self, record: TuneRecord) -> TuneRecord:
        self.records.append(record)
        return record

    def _recall(self, machine: str, key: str) -> dict | None:
        """This machine's stored answer for ``key``; None without a cache or an answer."""
        return self.cache.get(machine, key) if self.cache is not None else None

    def _remember(self, machine: str, key: str, entry: dict) -> None:
        if self.cache is not None:
            self.cache.put(machine, key, entry)

    def _cost(self, timers, progress=None):
        """``choose``'s cost function over ``timers`` [(timer, weight)]: each candidate's
        seconds per call under every timer, weighted and added (a generated kernel's decode
        and prefill workloads), over the stage's share of the tuner's rounds."""
        def cost(stage: str, candidates: list[int]) -> list[float]:
            rounds = self.rounds * ROUNDS_FACTOR[stage]
            total = np.zeros(len(candidates))
            for timer, weight in timers:
                total += weight * np.asarray(measure(timer, candidates, rounds, self.reps, progress))
            return [float(x) for x in total]
        return cost

    def tune_problem(self, make, op: str, shape: tuple, space: list[dict] | None) -> TuneRecord:
        """Answer one library problem: the schedule ``make()``'s problem should launch with.

        The candidates are ``space``, or the problem's own ``space()``. A stored
        answer for this machine is used as it is; otherwise every candidate's
        output is first compared bit for bit with schedule 0's inside guard
        regions (``problem.output``), and only then are they timed and chosen
        between (``choose``), the answer stored for next time.
        """
        began = time.perf_counter()
        problem = make() if space is None else None
        space = problem.space() if problem is not None else space
        key = self.problem_key(op, *((list(shape) + [0, 0, 0])[:3]), space, extra=tuple(shape[3:]))
        machine = machine_key()
        answer = self._recall(machine, key)
        if answer is not None and isinstance(answer.get("winner"), int):
            return self._log(TuneRecord(key, op, tuple(shape), len(space), answer["winner"],
                                        (answer.get("default_cost"), answer.get("winner_cost")), cached=True,
                                        seconds=time.perf_counter() - began))
        problem = problem if problem is not None else make()
        numbers = [c["schedule"] for c in space]
        incumbent = problem.output(numbers[0])
        for number in numbers[1:]:
            if not np.array_equal(problem.output(number), incumbent):
                raise TuningError(f"{op} schedule {number} on {tuple(shape)} differs from the default's bits")
        winner, trail, before, after = choose(numbers, self._cost([(problem, 1.0)]), self.margin)
        record = self._log(TuneRecord(key, op, tuple(shape), len(space), winner, (before, after),
                                      evaluations=tuple(trail), seconds=time.perf_counter() - began))
        self._remember(machine, key, {"winner": winner, "default_cost": before, "winner_cost": after,
                                      "op": op, "shape": list(shape)})
        if self.verbose:
            print(f"tuned {op} {tuple(shape)}: {len(space)} schedules in {record.seconds:.1f} s, "
                  f"schedule {winner} at {after * 1e6:.2f} us ({record.speedup:.2f}x the default)",
                  file=sys.stderr, flush=True)
        return record
