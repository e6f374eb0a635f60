"""The reference's recorded programs (tests/golden/programs.json.gz) and a restatement of its model driver.

TEST INFRASTRUCTURE. ``make_programs.py`` recorded, in the build container,
what the reference's compiler makes of a zoo of small graphs and of the
tiny golden Qwen2 (G5) in its three modes, with the reference's C outputs on
seeded inputs. The driver below restates the reference's ``Qwen2.forward``,
``KVCache`` and ``greedy`` (models/qwen2.py:232-368): the host cache handed
to each call as ``past_keys``/``past_values``, the new keys and values
appended after it, argmax decoding, so the recorded graphs can be driven
through any ``run(graph_name, inputs, weights)``.
"""

from __future__ import annotations

from functools import lru_cache
from pathlib import Path

import numpy as np

from nanocompile_amd import lir
from nanocompile_amd.models.config import TINY, TINY_STD, random_weights

GOLDEN = Path(__file__).resolve().parent / "golden"
TAGS = {"f32": None, "int8": "int8", "vnni": "int8-vnni"}
PROMPTS = ([4, 5, 6], [7, 8], [1], [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5])     # golden G5's

# Outputs computed through exp, sin or cos: the C library's and this package's
# differ by an ulp on rare inputs, so these are held to the reference's own
# tolerance for those functions (test_codegen.py:28-29); everything else is bitwise.
APPROX = {"unary": {"exp", "sin", "cos"}, "softmax_mask": {"p"}, "rope": {"y"}}
APPROX_PREFIX = ("mlp_",)
RTOL, ATOL = 2e-6, 1e-6


@lru_cache(maxsize=None)
def fixture():
    return lir.load_programs(GOLDEN / "programs.json.gz"), np.load(GOLDEN / "programs.npz", allow_pickle=False)


def zoo_names() -> list[str]:
    return sorted(fixture()[0]["zoo"])


def zoo(name: str, variant: str = "program") -> lir.Program:
    doc, arrays = fixture()
    return lir.program_from_json(doc["zoo"][name][variant], arrays)


def zoo_cases(name: str):
    """[(inputs, expected outputs or None, error text or None)] and the weights."""
    doc, arrays = fixture()
    entry = doc["zoo"][name]
    weights = {w: arrays[key] for w, key in entry["weights"].items()}
    cases = []
    for case in entry["cases"]:
        inputs = {k: arrays[v] for k, v in case["inputs"].items()}
        outputs = {k: arrays[v] for k, v in case["outputs"].items()} if "error" not in case else None
        cases.append((inputs, outputs, case.get("error")))
    return cases, weights


def approx(name: str) -> set[str]:
    if name.startswith(APPROX_PREFIX):
        return {"y"}
    return APPROX.get(name, set())


def qwen2(tag: str, which: str) -> lir.Program:
    doc, arrays = fixture()
    return lir.program_from_json(doc["qwen2"][tag][which], arrays)


def qwen2_weights(tag: str) -> dict[str, np.ndarray]:
    """The tiny model's weights as the reference hands them to its runner (quantize.py:167-180):
    float32 by name, and for each int8 projection ``W@int8`` / ``W@scales`` from the reference's
    per-row quantizer (restated in oracle/reference.py, pinned by golden G1)."""
    from oracle import reference as R
    doc, _ = fixture()
    names = doc["qwen2"][tag]["weight_names"]
    base = random_weights(TINY, seed=5, std=TINY_STD)
    out = {}
    for name in names:
        if name.endswith("@int8") or name.endswith("@scales"):
            w = name.rsplit("@", 1)[0]
            q, s = R.quantize_int8(base[w])
            out[name] = q if name.endswith("@int8") else s
        else:
            out[name] = base[name]
    return out


def config5() -> tuple[lir.Program, dict]:
    """Config 5's last-position forward program (Qwen2.5-0.5B-shaped, int8) as the reference
    compiles it, and what the fixture holds of the reference's run: the prompt, its greedy
    tokens, and logits of the prompt and of the first decode step at every ``stride``-th entry."""
    doc, arrays = fixture()
    entry = doc["config5"]
    record = {k: v for k, v in entry.items() if k != "last"}
    record["logits_prompt"] = arrays["config5/logits_prompt"]
    record["logits_step"] = arrays["config5/logits_step"]
    return lir.program_from_json(entry["last"], arrays), record


def config5_weights(names, seed: int) -> dict[str, np.ndarray]:
    """Config 5's seeded weights as the reference hands them to its runner: float32 by name, each
    int8 projection as ``W@int8`` / ``W@scales`` from the per-row quantizer (oracle/reference.py,
    pinned by golden G1)."""
    from nanocompile_amd.models.config import QWEN25_05B
    from oracle import reference as R
    base = random_weights(QWEN25_05B, seed=seed)
    out = {}
    for name in names:
        if name.endswith("@int8"):
            w = name.rsplit("@", 1)[0]
            out[name], out[w + "@scales"] = R.quantize_int8(base[w])
        elif not name.endswith("@scales"):
            out[name] = base[name]
    return out


class Driver:
    """The reference's Qwen2 forward and greedy loop over a runner ``run(which, inputs) -> outputs``,
    ``which`` being "full" or "last" (models/qwen2.py:316-368)."""

    def __init__(self, run, config=TINY) -> None:
        self.run, self.config = run, config

    def empty(self) -> tuple[np.ndarray, np.ndarray]:
        c = self.config
        z = np.zeros((c.num_hidden_layers, c.num_key_value_heads, 0, c.head_dim), np.float32)
        return z, z

    def forward(self, ids, cache=None, last_only=False) -> np.ndarray:
        ids = np.asarray(ids, np.int64)
        past_keys, past_values = cache if cache is not None else self.empty()
        out = self.run("last" if last_only else "full",
                       {"token_ids": ids, "past_keys": past_keys, "past_values": past_values})
        if cache is not None:
            cache[0] = np.concatenate([cache[0], out["keys"]], axis=2)
            cache[1] = np.concatenate([cache[1], out["values"]], axis=2)
        return out["logits"]

    def greedy(self, prompt, n: int) -> list[int]:
        cache = list(self.empty())
        pending, out = list(prompt), []
        for _ in range(n):
            token = int(np.argmax(self.forward(pending, cache, last_only=True)[0]))
            out.append(token)
            pending = [token]
        return out


def candidate_programs() -> list[tuple[str, str]]:
    """(zoo name, variant) of the programs whose every schedule candidate the GPU tests run and
    tune: each zoo graph as fused, and config 2's graph unfused (a kernel per operation)."""
    return [(n, "program") for n in zoo_names()] + [("rms_norm_quant", "unfused")]


def candidate_models() -> list[tuple[str, str]]:
    """(mode, which) of the tiny Qwen2 programs the GPU tests tune (every kernel's candidates)."""
    return [("int8", "full"), ("int8", "last")]


def prebuild(jobs: int = 8) -> int:
    """Build every recorded program's library (default GPU schedules), and the candidate
    libraries of ``candidate_programs`` (every schedule of every kernel), into the codegen cache,
    in parallel, so that GPU runs find them built; returns how many were compiled afresh."""
    from concurrent.futures import ThreadPoolExecutor

    from nanocompile_amd import autotune, codegen_hip, compiled
    doc, _ = fixture()
    progs = [zoo(n, v) for n in zoo_names() for v in ("program", "unfused", "scheduled")]
    progs += [qwen2(tag, which) for tag, entry in doc["qwen2"].items() for which in entry if which != "weight_names"]
    progs.append(config5()[0])
    libraries = [autotune.CandidateLibrary(zoo(n, v)) for n, v in candidate_programs()]
    libraries += [autotune.CandidateLibrary(qwen2(tag, which)) for tag, which in candidate_models()]
    libraries.append(autotune.CandidateLibrary(config5()[0]))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(compiled.prebuild, progs))
        results.append(compiled.prebuild(lane_store_program(), lane_store_lanes))
        results.append(compiled.prebuild(lane_store_program()))
        results += list(pool.map(lambda library: library.build(), libraries))
    # libraries of sources no longer generated would only travel to the GPU with the tree
    keep = {path.name for path, _ in results}
    for stale in codegen_hip.cache_dir().glob("nc_hip_*.so"):
        if stale.name not in keep:
            stale.unlink()
    return sum(1 for _, cached in results if not cached)


def lane_store_program(rows: int = 3, width: int = 8, steps: int = 4) -> lir.Program:
    """A hand-built program whose item stores its accumulators directly, ``y[i, e] = acc[e]``:
    ``acc[e] = fma(x[i, s * width + e], 2, acc[e])`` over ``steps``, then one store per element.
    Held across lanes, element e lives in lane e, so the store's value is a shuffle that every
    lane must take part in while only lane 0 stores. Returns the program; its input is ``x``
    [rows, steps * width] float32 and its output ``y`` [rows, width]."""
    f32, i64 = lir.DType("f32"), lir.DType("i64")

    def c(x):
        return lir.Const(x, i64)

    def add(a, b):
        return lir.Binary("add", a, b, i64)

    def mul(a, b):
        return lir.Binary("mul", a, b, i64)

    k = steps * width
    i, s, e = lir.Var("i0"), lir.Var("k0"), lir.Var("e0")
    chain = lir.Loop("k0", c(steps), (lir.Loop("kl", c(width), (lir.ArrayStore("acc", lir.Var("kl"), lir.Fma(
        lir.Load(1, add(add(mul(i, c(k)), mul(s, c(width))), lir.Var("kl")), f32), lir.Const(2.0, f32),
        lir.Local("acc", lir.Var("kl"), f32), f32)),), "serial"),), "serial")
    store = lir.Loop("e0", c(width), (lir.Store(0, add(mul(i, c(width)), e), lir.Local("acc", e, f32)),), "serial")
    kernel = lir.Kernel("lane_store", (lir.Param(f32, True), lir.Param(f32, False)), (lir.Loop("i0", c(rows), (
        lir.Array("acc", width, lir.Const(0.0, f32)), chain, store), "parallel"),))
    x = lir.Buffer("input", f32, (rows, k), "x")
    y = lir.Buffer("output", f32, (rows, width), "y")
    call = lir.Call(0, y, (lir.View(x, (rows, k), (k, 1), 0),), "lane_store", 0)
    return lir.Program("lane_store", (), [("x", f32, (rows, k))], {}, [kernel], [call], [x, y], {"y": y})


def lane_store_lanes(kernel, calls):
    """``lane_store_program``'s kernel with its accumulators one element a lane."""
    from nanocompile_amd import gpu_schedule
    s = gpu_schedule.GpuSchedule(kernel).grid("i0").lanes("acc")
    return s.kernel, s.launch


def lane_store_expected(x: np.ndarray, width: int = 8) -> np.ndarray:
    """``lane_store_program``'s output computed directly: each element's chain of fused
    multiply-adds in order. For float32 x and acc of normal magnitudes, 2 x + acc is exact in
    float64, so rounding it to float32 once is what the fused multiply-add gives."""
    rows, k = x.shape
    acc = np.zeros((rows, width), np.float32)
    for s in range(k // width):
        acc = (x[:, s * width:(s + 1) * width].astype(np.float64) * 2.0 + acc.astype(np.float64)).astype(np.float32)
    return acc
